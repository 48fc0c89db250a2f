"""Hybrid-attention DiT block forward on gfx950 kernels (MXFP8 GEMMs, window softmax, VDA).

Composition (reference: src/models/ops/fused_block.py:134-169 paper_block_forward with fused
producers; src/inference/utils/tensor_parallel.py:169-228 tp_attention_forward at world size
1; src/models/hybrid_attention.py:178-255; src/inference/utils/paper_adaln.py:174-188 AdaLN
tables; src/inference/utils/lora.py:80-107 LoRA merge):

  shift/scale/gate (attn, mlp) = Linear(SiLU(temb.float()).to(bf16))            6 x [1, H]
  x1, q1 = prenorm-quantize(h; norm1, scale_msa, shift_msa)                       bf16 + MXFP8
  qkv    = MXFP8 GEMM(q1, W_qkv + B_lora A_lora)                                  [T, 3H]
  gates  = sigmoid(softmax_gate(x1)), beta = sigmoid(beta_proj(x1)),
           lin_gate = sigmoid(up(down(x1))), alpha = FrameKDAAlpha(frame mean of x1)
           (one bf16 MFMA pass over x1 for the gate, beta, down and alpha-down columns,
           vdn_gate_projection; the alpha MLP on per-frame column sums, vdn_frame_alpha)
  soft   = window attention(QK-RMSNorm + 3D RoPE(q, k), v) * gate                 [T, H]
  far    = VDA(raw q, k, v, beta, lin_gate, alpha)                                [T, H]
  h      = h + gate_msa * [O | O_lin]([soft | far])          one K = 2H GEMM, residual fused
  h      = h + O_c(cross attention(RMSNorm3(h) -> q, context -> k, v))
  x2, q2 = prenorm-quantize(h; norm2, scale_mlp, shift_mlp)
  h      = h + gate_mlp * down(GELU-tanh(up(q2)))           GELU + MXFP8 in the up GEMM epilogue

The GELU-tanh FFN and the cross-attention have no reference kernel (the reference block uses
SwiGLU and packs text into the sequence); they follow the torch definitions (GELU
approximate='tanh'; cross-attention = QK-RMSNorm'd SDPA over the context rows, unmasked).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from . import mxfp8 as mx
from . import vda as vv
from . import window as vw

GATE_GROUP = 64      # softmax-gate / beta columns of the gate projection (heads <= 64)
GATE_ROWS = 128      # rows per gate-projection workgroup (per-frame partial sums)


def gate_weight(w: "BlockWeights", cfg: "BlockConfig") -> torch.Tensor:
    """[384, hidden] bf16 operand of vdn_gate_projection: softmax-gate rows, beta rows (each
    group zero-padded to 64), output-gate down (128) and FrameKDAAlpha down (128). An odd head
    count runs as the next even one (the kernel stores head pairs): the extra gate and beta
    rows are the zero padding, and gate_projection drops their columns."""
    if cfg.heads + cfg.heads % 2 > GATE_GROUP or cfg.head_dim != 128 or cfg.hidden % 32:
        raise NotImplementedError("the gate projection needs at most 64 heads (63 if odd), "
                                  "head_dim 128 and hidden % 32 == 0")
    out = torch.zeros(2 * GATE_GROUP + 256, cfg.hidden, dtype=torch.bfloat16,
                      device=w.soft_gate_w.device)
    out[:cfg.heads] = w.soft_gate_w
    out[GATE_GROUP:GATE_GROUP + cfg.heads] = w.beta_w
    out[2 * GATE_GROUP:2 * GATE_GROUP + 128] = w.lgate_down_w
    out[2 * GATE_GROUP + 128:] = w.alpha_down_w
    return out


def gate_projection(x1, weight, gate_bias, heads, frames, spatial):
    """soft_gate [T, heads], beta [T, heads], gate_down [T, 128] (bf16) and the per-frame
    column sums of x1 @ alpha_down^T [frames * ceil(spatial / 128), 128] (fp32) of x1
    [frames * spatial, hidden] bf16 (attention_gates.py:52-55, tensor_parallel.py:194-198).
    An odd head count runs the kernel on heads + 1 columns (weight rows `heads` of the gate
    and beta groups are zero in gate_weight, the bias gets a zero) and returns the first
    `heads` columns."""
    t, hd = x1.shape
    for name, ten in (("x1", x1), ("weight", weight), ("gate_bias", gate_bias)):
        _lib.require_gpu(ten, name)
        if ten.dtype != torch.bfloat16 or ten.device != x1.device:
            raise ValueError(f"{name} must be bf16 on the device of x1")
    if t != frames * spatial or x1.stride(1) != 1:
        raise ValueError("x1 must be [frames * spatial, hidden] with unit column stride")
    if weight.shape != (2 * GATE_GROUP + 256, hd) or not weight.is_contiguous():
        raise ValueError("weight must be the contiguous [384, hidden] gate_weight operand")
    if gate_bias.numel() < heads or not gate_bias.is_contiguous():
        raise ValueError("gate_bias must be contiguous with heads entries")
    dev = x1.device
    odd = heads % 2
    if odd:
        if heads + 1 > GATE_GROUP:
            raise ValueError("an odd head count must be below 64")
        gate_bias = torch.cat((gate_bias.reshape(-1)[:heads],
                               torch.zeros(1, dtype=torch.bfloat16, device=dev)))
    hk = heads + odd
    soft = torch.empty(t, hk, dtype=torch.bfloat16, device=dev)
    beta = torch.empty(t, hk, dtype=torch.bfloat16, device=dev)
    down = torch.empty(t, 128, dtype=torch.bfloat16, device=dev)
    bpf = -(-spatial // GATE_ROWS)
    partial = torch.empty(frames * bpf, 128, dtype=torch.float32, device=dev)
    _lib.call("vdn_gate_projection", x1.data_ptr(), x1.stride(0), hd, weight.data_ptr(), hk,
              frames, spatial, gate_bias.data_ptr(), soft.data_ptr(), beta.data_ptr(),
              down.data_ptr(), partial.data_ptr(), _lib.stream(dev))
    if odd:
        soft, beta = soft[:, :heads].contiguous(), beta[:, :heads].contiguous()
    return soft, beta, down, partial


def frame_alpha(partial, frames, spatial, up_w, dt_bias, a_log, heads, head_dim):
    """FrameKDAAlpha (layers.py:36-69) from the gate projection's per-frame sums: alpha
    [frames, heads, head_dim] fp32 = exp(-exp(A_log) softplus(up(mean) + dt_bias))."""
    for name, t, dt in (("partial", partial, torch.float32), ("up_w", up_w, torch.bfloat16),
                        ("dt_bias", dt_bias, torch.float32), ("a_log", a_log, torch.float32)):
        _lib.require_gpu(t, name)
        if t.dtype != dt or not t.is_contiguous() or t.device != partial.device:
            raise ValueError(f"{name} must be contiguous {dt} on the device of partial")
    if partial.shape != (frames * -(-spatial // GATE_ROWS), 128):
        raise ValueError("partial must be the gate projection's [frames * blocks, 128] sums")
    if dt_bias.numel() != heads * head_dim or a_log.numel() != heads:
        raise ValueError("dt_bias must have heads * head_dim entries and a_log heads")
    if up_w.shape != (heads * head_dim, 128):
        raise ValueError("up_w must be [heads * head_dim, 128]")
    alpha = torch.empty(frames, heads, head_dim, dtype=torch.float32, device=partial.device)
    _lib.call("vdn_frame_alpha", partial.data_ptr(), frames, spatial, up_w.data_ptr(),
              dt_bias.data_ptr(), a_log.data_ptr(), heads, head_dim, alpha.data_ptr(),
              _lib.stream(partial.device))
    return alpha


def adaln_tables(temb, weight, bias, hidden):
    """Six [m, hidden] bf16 tables Linear(bf16(SiLU(temb in fp32)), weight, bias) in the order
    shift, scale, gate (attention), shift, scale, gate (MLP) (paper_adaln.py:174-188). The
    kernel reads bf16 or fp32 temb and runs SiLU in fp32; any other floating dtype is taken
    through temb.float() first, as the reference's SiLU(temb.float()) does (exact for fp16)."""
    if temb.dtype not in (torch.bfloat16, torch.float32):
        if not temb.dtype.is_floating_point:
            raise ValueError("temb must be a floating-point tensor")
        temb = temb.float()
    _lib.require_gpu(temb, "temb")
    for name, t in (("weight", weight),) + ((("bias", bias),) if bias is not None else ()):
        _lib.require_gpu(t, name)
        if t.dtype != torch.bfloat16 or t.device != temb.device:
            raise ValueError(f"{name} must be bf16 on the device of temb")
    if temb.dim() != 2 or temb.stride(1) != 1:
        raise ValueError("temb must be [m, hidden] with unit column stride")
    if weight.shape != (6 * hidden, temb.shape[1]) or not weight.is_contiguous():
        raise ValueError("weight must be contiguous [6 * hidden, hidden]")
    if bias is not None and (bias.numel() != 6 * hidden or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous with 6 * hidden entries")
    m = temb.shape[0]
    out = torch.empty(m, 6 * hidden, dtype=torch.bfloat16, device=temb.device)
    _lib.call("vdn_adaln_tables", temb.data_ptr(), int(temb.dtype == torch.float32),
              temb.stride(0), m, temb.shape[1],
              weight.data_ptr(), bias.data_ptr() if bias is not None else None, 6 * hidden,
              out.data_ptr(), out.stride(0), _lib.stream(temb.device))
    return out.chunk(6, dim=-1)


@dataclass(frozen=True)
class BlockConfig:
    """Block widths. The attention width heads * head_dim may differ from the hidden width
    (VDN-H3: hidden 5376, 56 x 128 heads). ffn_act "gelu_tanh" (up: hidden -> ffn) or
    "swiglu" (VDN-H3, mxfp8_kernels.py:62-64: up: hidden -> 2 ffn = [a | g], a * silu(g))."""
    hidden: int = 5120
    heads: int = 40
    head_dim: int = 128
    ffn: int = 13824
    ffn_act: str = "gelu_tanh"
    context: int = 512
    lora_rank: int = 64
    lora_scale: float = 1.0
    eps: float = 1e-6
    radius: int = 1
    rope_dims: tuple = (44, 42, 42)
    rope_theta: float = 10000.0
    vda_chunk: int = 8
    init_std: float = 0.02

    @property
    def inner(self) -> int:
        """Attention width: heads * head_dim."""
        return self.heads * self.head_dim

    @property
    def ffn_up(self) -> int:
        """Output width of the FFN's up projection."""
        return 2 * self.ffn if self.ffn_act == "swiglu" else self.ffn


@dataclass
class BlockWeights:
    """bf16 master weights of one block (random init), the source of both the MXFP8
    buffers and the oracle."""
    tensors: dict

    def __getattr__(self, name):
        try:
            return self.tensors[name]
        except KeyError as e:
            raise AttributeError(name) from e

    @staticmethod
    def random(cfg: BlockConfig, seed: int = 0, device="cpu") -> "BlockWeights":
        if cfg.ffn_act not in ("gelu_tanh", "swiglu"):
            raise ValueError("ffn_act must be gelu_tanh or swiglu")
        g = torch.Generator(device=device).manual_seed(seed)
        hd, h, n, f, r = cfg.hidden, cfg.heads, cfg.head_dim, cfg.ffn, cfg.lora_rank
        inner, fu = cfg.inner, cfg.ffn_up

        def normal(*shape, std=cfg.init_std):
            return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

        def ones_ish(size):
            return (1.0 + torch.randn(size, generator=g, device=device) * 0.1).to(torch.bfloat16)

        a = torch.empty(h, device=device).uniform_(1, 16, generator=g)
        dt = torch.exp(torch.rand(h * n, generator=g, device=device)
                       * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp(min=1e-4)
        t = dict(
            adaln_w=normal(6 * hd, hd), adaln_b=normal(6 * hd),
            norm1=ones_ish(hd), norm2=ones_ish(hd), norm3=ones_ish(hd),
            qkv_w=normal(3 * inner, hd), qkv_b=normal(3 * inner),
            lora_a=normal(3, r, hd), lora_b=normal(3, inner, r),
            norm_q=ones_ish(n), norm_k=ones_ish(n),
            o_w=normal(hd, inner), o_b=normal(hd), olin_w=normal(hd, inner),
            soft_gate_w=normal(h, hd), soft_gate_b=normal(h),
            beta_w=normal(h, hd),
            lgate_down_w=normal(n, hd), lgate_up_w=normal(inner, n), lgate_up_b=normal(inner),
            alpha_down_w=normal(n, hd), alpha_up_w=normal(inner, n),
            a_log=torch.log(a).float(), dt_bias=(dt + torch.log(-torch.expm1(-dt))).float(),
            vda_norm=ones_ish(n),
            cq_w=normal(inner, hd), cq_b=normal(inner), ck_w=normal(inner, hd), ck_b=normal(inner),
            cv_w=normal(inner, hd), cv_b=normal(inner), co_w=normal(hd, inner), co_b=normal(hd),
            norm_qc=ones_ish(n), norm_kc=ones_ish(n),
            up_w=normal(fu, hd), up_b=normal(fu), down_w=normal(hd, f), down_b=normal(hd),
        )
        return BlockWeights(t)

    def merged_qkv(self, scale: float) -> torch.Tensor:
        """W_qkv with the rank-r LoRA of Q, K, V folded in: W += bf16(scale * (B @ A) in fp32)
        (lora.py:105-107)."""
        inner = self.qkv_w.shape[0] // 3
        w = self.qkv_w.clone()
        for i in range(3):
            delta = (self.lora_b[i].float() @ self.lora_a[i].float()) * scale
            w[i * inner:(i + 1) * inner].add_(delta.to(w.dtype))
        return w


def _linear(weight, bias=None):
    lin = nn.Linear(weight.shape[1], weight.shape[0], bias=bias is not None, device=weight.device,
                    dtype=weight.dtype)
    with torch.no_grad():
        lin.weight.copy_(weight)
        if bias is not None:
            lin.bias.copy_(bias)
    return lin


class HybridDiTBlock(nn.Module):
    """One hybrid DiT block; every projection in the attention/FFN path is an MXFP8Linear."""

    def __init__(self, cfg: BlockConfig, weights: BlockWeights):
        super().__init__()
        self.cfg = cfg
        w = weights
        mk = lambda weight, bias=None: mx.MXFP8Linear(_linear(weight, bias), check_finite=False)
        self.qkv = mk(w.merged_qkv(cfg.lora_scale), w.qkv_b)
        # to_out and to_out_linear share one GEMM over the concatenated branch outputs
        self.o_cat = mk(torch.cat((w.o_w, w.olin_w), dim=1), w.o_b)
        self.cq, self.ck, self.cv, self.co = (mk(w.cq_w, w.cq_b), mk(w.ck_w, w.ck_b),
                                              mk(w.cv_w, w.cv_b), mk(w.co_w, w.co_b))
        if cfg.ffn_act == "swiglu":   # [a | g] interleaved for the fused SwiGLU producer
            self.up = mx.MXFP8Linear.swiglu_up(_linear(w.up_w, w.up_b), check_finite=False)
        else:
            self.up = mk(w.up_w, w.up_b)
        self.down = mk(w.down_w, w.down_b)
        # softmax gate | beta | output-gate down | alpha down: one pass over x1
        self.gate_w = gate_weight(w, cfg)
        self.keep = {k: w.tensors[k] for k in (
            "adaln_w", "adaln_b", "norm1", "norm2", "norm3", "norm_q", "norm_k", "soft_gate_b",
            "lgate_up_w", "lgate_up_b", "alpha_down_w", "alpha_up_w", "a_log", "dt_bias",
            "vda_norm", "norm_qc", "norm_kc")}
        self._zero_table = None
        self._zero_idx = None
        self._side = None
        # The VDA branch runs on a side stream beside RoPE + window attention; False runs it
        # after them on the caller's stream (same kernels, same outputs), which gives each
        # branch kernel an unshared launch time.
        self.overlap_vda = True

    # ---------------------------------------------------------------- pieces ----
    def adaln_tables(self, temb):
        """6 tables [1, H]: shift/scale/gate attention, then MLP (paper_adaln.py:174-188, 205-212)."""
        k = self.keep
        return adaln_tables(temb, k["adaln_w"], k["adaln_b"], self.cfg.hidden)

    def _side_stream(self, device):
        """One side stream per device, default priority."""
        if self._side is None or self._side.device != device:
            self._side = torch.cuda.Stream(device=device)
        return self._side

    def _zeros(self, device):
        if self._zero_table is None or self._zero_table.device != device:
            self._zero_table = torch.zeros(1, self.cfg.hidden, dtype=torch.bfloat16, device=device)
        return self._zero_table

    def _table_index(self, rows, device):
        """Row -> table index (all rows use table 0), kept between calls."""
        z = self._zero_idx
        if z is None or z.device != device or z.shape[0] < rows:
            self._zero_idx = z = torch.zeros(rows, dtype=torch.long, device=device)
        return z[:rows]

    # --------------------------------------------------------------- forward ----
    @torch.no_grad()
    def forward(self, hidden, temb, context, layout: vw.SequenceLayout, rope, window_plan,
                cross_plan, return_parts=False, guard=None):
        """hidden [T, H] bf16 (video rows), temb [1, H], context [L, H] bf16; rope = (cos, sin)
        [T, 128]; window_plan from prepare_paper_window_plan; cross_plan from cross_attention_plan.
        Returns the new hidden [T, H] (a fresh tensor); with return_parts also a dict of
        intermediate copies (tables, x1, qkv, soft, far, h1, co, h2) for checking.

        guard: an object with predicate(parts) (the reference's CoordinatedFiniteGuard,
        paper_runtime.py:43-50, or FinitePredicate below). Each MXFP8 producer's finite
        predicate is handed to it as a device bool tensor, as paper_block_forward does
        (fused_block.py:144-155): the three prenorm producers' per-row flags and, last, one
        flag for every projection output (q, k, v and the gated residuals in bf16, the FFN
        activation before its quantization). The branch outputs are quantized in their kernels
        and reach the [O | O_lin] projection, whose output carries any inf/NaN they hold.
        Nothing is read on the host."""
        cfg, k = self.cfg, self.keep
        T, hd = hidden.shape
        heads, d = cfg.heads, cfg.head_dim
        inner = cfg.inner
        frames, spatial = layout.num_frames, layout.tokens_per_frame
        dev = hidden.device
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaln_tables(temb)
        idx = self._table_index(T, dev)
        parts = {} if return_parts else None
        nf = None if guard is None else torch.zeros(1, dtype=torch.int32, device=dev)

        def producer(finite):
            if guard is not None:
                guard.predicate(finite)

        def snap(name, t):
            if parts is not None:
                parts[name] = t.clone() if isinstance(t, torch.Tensor) else t

        # ---- hybrid self-attention ----
        x1, q1, s1, fin = mx.launch_prenorm_quantize(hidden, k["norm1"], cfg.eps, scale_msa,
                                                     shift_msa, idx, write_bf16=True)
        producer(fin)
        qkv = self.qkv.forward_quantized(q1, s1, rows=T, nonfinite=nf)
        snap("tables", (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp))
        snap("x1", x1)
        snap("qkv", qkv)
        raw_q = qkv[:, :inner].view(T, heads, d)
        raw_k = qkv[:, inner:2 * inner].view(T, heads, d)
        value = qkv[:, 2 * inner:].view(T, heads, d)
        cos, sin = rope
        main = torch.cuda.current_stream(dev)
        side = self._side_stream(dev) if (self.overlap_vda and parts is None) else None

        def gates(ready=None):
            soft_gate, beta, gate_down, partial = gate_projection(
                x1, self.gate_w, k["soft_gate_b"], heads, frames, spatial)
            if ready is not None:   # the softmax gate exists: the attention may start
                ready.record()
            # the low-rank gate sigmoid(up(down(x1))) is formed inside the VDA readout
            lin_gate = vv.OutputGateProjection(gate_down, k["lgate_up_w"], k["lgate_up_b"])
            alpha = frame_alpha(partial, frames, spatial, k["alpha_up_w"], k["dt_bias"],
                                k["a_log"], heads, d)
            return soft_gate, beta, lin_gate, alpha

        def context_kv():
            """Context K (RMSNorm'd) and V of the cross-attention: they depend on the context
            rows only, so the overlapped schedule computes them on the side stream."""
            cx, csx = mx.launch_quantize(context)
            L = context.shape[0]
            ck = self.ck.forward_quantized(cx, csx, rows=L, nonfinite=nf).view(L, heads, d)
            cv = self.cv.forward_quantized(cx, csx, rows=L, nonfinite=nf).view(L, heads, d)
            return vw.qk_rmsnorm(ck, k["norm_kc"], cfg.eps), cv

        if side is not None:
            # The gate projection (x1 only) runs on the side stream beside the QK norm + RoPE
            # pass; the window attention waits for its softmax gate through an event.
            side.wait_stream(main)
            gate_ready = torch.cuda.Event()
            with torch.cuda.stream(side):
                soft_gate, beta, lin_gate, alpha = gates(gate_ready)
        else:
            soft_gate, beta, lin_gate, alpha = gates()
        # The two branch outputs are the two halves of the [O | O_lin] operand. The kernels
        # quantize them in their epilogues straight into the MXFP8 operand (chunks 0..H-1 for
        # the softmax branch, H.. for VDA); with return_parts they are kept in bf16 for the
        # snapshots and quantized afterwards, which gives the same bytes.
        bounds = window_plan.bounds
        if parts is None:
            qb, sb = mx.empty_activation(T, 2 * inner, dev)

            def linear_branch():
                vv.vda_forward(raw_q, raw_k, value, beta, lin_gate, alpha, bounds,
                               frames, spatial, k["vda_norm"], cfg.eps, chunk_size=cfg.vda_chunk,
                               out_mxfp8=(qb, sb, heads))

            # The VDA branch runs on a side stream while RoPE and the window attention run on
            # the caller's stream (the reference's paper_vda_overlap, tensor_parallel.py:
            # 202-216): its latency-bound passes fill the attention's gaps. The context K and V
            # of the cross-attention follow it there. The tensors the side stream shares with
            # the caller's stream (x1, qkv, the gates, alpha, the [O | O_lin] operand, the
            # context K and V) are all released after main.wait_stream(side), so a later
            # allocation on the caller's stream is ordered after the branch without
            # record_stream (which would keep ~5 GB per block out of the allocator's cache
            # while the host runs ahead); a side-stream allocation is ordered after them by
            # the next side.wait_stream(main).
            if side is not None:
                with torch.cuda.stream(side):
                    linear_branch()
                    ck, cv = context_kv()
            q, kk = vw.paper_qk_rmsnorm_rope(raw_q, raw_k, k["norm_q"], k["norm_k"], cfg.eps,
                                             cos, sin, enabled=True)
            if side is not None:
                main.wait_event(gate_ready)
            vw.paper_window_attention(q, kk, value, window_plan, d ** -0.5, enabled=True,
                                      gate=soft_gate, out_mxfp8=(qb, sb, 0))
            del q, kk
            if side is not None:
                main.wait_stream(side)
            else:
                linear_branch()
        else:
            q, kk = vw.paper_qk_rmsnorm_rope(raw_q, raw_k, k["norm_q"], k["norm_k"], cfg.eps,
                                             cos, sin, enabled=True)
            both = torch.empty((T, 2 * inner), dtype=torch.bfloat16, device=dev)
            vw.paper_window_attention(q, kk, value, window_plan, d ** -0.5, enabled=True,
                                      gate=soft_gate, out=both[:, :inner].view(T, heads, d))
            del q, kk
            vv.vda_forward(raw_q, raw_k, value, beta, lin_gate, alpha, bounds,
                           frames, spatial, k["vda_norm"], cfg.eps, chunk_size=cfg.vda_chunk,
                           out=both[:, inner:])
            snap("soft", both[:, :inner])
            snap("far", both[:, inner:])
            qb, sb = mx.launch_quantize(both)
            del both
        del qkv, raw_q, raw_k, value, lin_gate, soft_gate, beta, alpha
        # the first residual update writes a fresh tensor (no copy of the input)
        h = torch.empty_like(hidden)
        self.o_cat.forward_quantized(qb, sb, rows=T, out=h, residual=hidden, gate=gate_msa,
                                     nonfinite=nf)
        snap("h1", h)
        del qb, sb

        # ---- cross-attention to the context rows ----
        zeros = self._zeros(dev)
        _, q3, s3, fin = mx.launch_prenorm_quantize(h, k["norm3"], cfg.eps, zeros, zeros, idx,
                                                    write_bf16=False)
        producer(fin)
        cq = self.cq.forward_quantized(q3, s3, rows=T, nonfinite=nf).view(T, heads, d)
        if side is None:
            ck, cv = context_kv()
        if parts is None:
            # the queries' RMSNorm runs in the attention kernel as it loads them
            qo, so = mx.empty_activation(T, inner, dev)
            cross_attention(cq, ck, cv, cross_plan, d ** -0.5, out_mxfp8=(qo, so, 0),
                            q_norm=(k["norm_qc"], cfg.eps))
        else:
            cq = vw.qk_rmsnorm(cq, k["norm_qc"], cfg.eps)
            co = cross_attention(cq, ck, cv, cross_plan, d ** -0.5)
            snap("co", co.view(T, inner))
            qo, so = mx.launch_quantize(co.view(T, inner))
            del co
        del cq, ck, cv
        self.co.forward_quantized(qo, so, rows=T, out=h, residual=h, nonfinite=nf)
        del qo, so
        snap("h2", h)

        # ---- FFN ----
        _, q4, s4, fin = mx.launch_prenorm_quantize(h, k["norm2"], cfg.eps, scale_mlp,
                                                    shift_mlp, idx, write_bf16=False)
        producer(fin)
        # up + activation + MXFP8 in the GEMM's epilogue (for SwiGLU the [a | g] halves meet
        # in it: tp_ff_forward's project + launch_swiglu_quantize, tensor_parallel.py:147-161)
        q5, s5 = self.up.forward_act_quantized(q4, s4, rows=T, act=cfg.ffn_act, nonfinite=nf)
        snap("ffn_codes", (q5, s5))
        self.down.forward_quantized(q5, s5, rows=T, out=h, residual=h, gate=gate_mlp,
                                    nonfinite=nf)
        if guard is not None:
            guard.predicate(nf == 0)
        return (h, parts) if return_parts else h


class FinitePredicate:
    """A single-GPU finite guard with the reference guard's predicate seam
    (CoordinatedFiniteGuard.predicate / check, paper_runtime.py:43-50, 71-117, without the
    multi-rank vote): predicate() folds a device bool tensor into one device flag with no
    host sync; check() is the one explicit host read and raises FloatingPointError."""

    def __init__(self, device):
        self.pending = torch.ones((), dtype=torch.bool, device=device)

    def predicate(self, parts: torch.Tensor) -> None:
        self.pending.logical_and_(parts.all())

    def check(self, label: str) -> None:
        ok = bool(self.pending.item())
        self.pending.fill_(True)
        if not ok:
            raise FloatingPointError(f"nonfinite value before {label}")


def cross_attention_plan(num_queries: int, num_keys: int, device) -> vw.DevicePlan:
    """Every query sees every context key: one group, one key interval [0, num_keys)."""
    return vw._device_plan([(((0, num_queries),), ((0, num_keys),))], torch.device(device))


def cross_attention(q, k, v, plan: vw.DevicePlan, scale, out_mxfp8=None, q_norm=None):
    """Unmasked attention of q [T, H, D] over context k, v [L, H, D] on the window kernel.
    `out_mxfp8` = (codes, scales, chunk0): quantize the output in the kernel (head h -> chunk
    chunk0 + h) instead of returning bf16 [T, H, D]. With it, `q_norm` = (weight [D], eps)
    applies the queries' RMSNorm (vw.qk_rmsnorm) first, in the kernel as it loads them for a
    bf16 weight (the same bits as the separate pass), else as that pass."""
    from . import _lib
    T, h, d = q.shape
    if q_norm is not None and out_mxfp8 is None:
        raise ValueError("q_norm is fused into the MXFP8-output form only")
    if out_mxfp8 is not None:
        codes, scales, chunk0 = mx.mxfp8_destination(out_mxfp8, T, h, q.device)
        qw, qeps = (None, 0.0) if q_norm is None else q_norm
        if qw is not None:
            if qw.shape != (d,) or qw.device != q.device:
                raise ValueError("q_norm weight must be a [head_dim] tensor on q's device")
            if qw.dtype != torch.bfloat16 or qw.data_ptr() % 16:
                q, qw = vw.qk_rmsnorm(q, qw, qeps), None
        _lib.call("vdn_window_attention_mxfp8", q.data_ptr(), q.stride(0), q.stride(1),
                  k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
                  plan.blocks.data_ptr(), plan.nblocks, plan.intervals.data_ptr(),
                  plan.counts.data_ptr(), h, float(scale), None, 0, 0, _lib.ptr(qw),
                  float(qeps), codes.data_ptr(), scales.data_ptr(), codes.shape[1], chunk0,
                  _lib.stream(q.device))
        return None
    out = torch.empty_like(q)
    _lib.call("vdn_window_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
              k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
              plan.blocks.data_ptr(), plan.nblocks, plan.intervals.data_ptr(),
              plan.counts.data_ptr(), h, d, 0, float(scale), None, 0, 0, out.data_ptr(),
              out.stride(0), out.stride(1), None, 0, 0, _lib.stream(q.device))
    return out


def make_inputs(cfg: BlockConfig, frames: int, height: int, width: int, seed: int = 1,
                device="cpu"):
    """Synthetic block inputs: hidden ~ N(0,1) bf16 [F*h*w, H], temb ~ N(0,1) [1, H],
    context ~ N(0,1) bf16 [cfg.context, H]; 3D RoPE tables; +-radius frame window plan."""
    g = torch.Generator(device=device).manual_seed(seed)
    T = frames * height * width
    hidden = torch.randn(T, cfg.hidden, generator=g, device=device).to(torch.bfloat16)
    temb = torch.randn(1, cfg.hidden, generator=g, device=device)
    context = torch.randn(cfg.context, cfg.hidden, generator=g, device=device).to(torch.bfloat16)
    layout = vw.SequenceLayout(T, 0, frames, height * width, frame_height=height, frame_width=width)
    cos, sin = vw.rope_tables_3d(frames, height, width, dims=cfg.rope_dims, theta=cfg.rope_theta,
                                 device=device, dtype=torch.bfloat16)
    return hidden, temb, context, layout, (cos, sin)
