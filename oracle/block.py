"""Hybrid DiT block oracle: the block composition on the CPU. TEST INFRASTRUCTURE ONLY.

Composition (reference: src/models/ops/fused_block.py:43-51 _pre_ref/_post_ref and :134-169
paper_block_forward; src/inference/utils/paper_adaln.py:174-188 AdaLN tables;
src/inference/utils/tensor_parallel.py:169-228 attention at world size 1;
src/models/hybrid_attention.py:178-255 softmax + VDA branches; src/inference/utils/lora.py:80-107
LoRA merge; src/models/attention_gates.py:52-55 output gate; src/models/linear_attention/
layers.py:36-69 FrameKDAAlpha). The GELU-tanh FFN and the cross-attention to context rows have
no reference kernel: they follow the torch definitions (nn.GELU(approximate='tanh'); SDPA of
QK-RMSNorm'd queries over all context keys) and their parity is unpinned against the reference.

Every MXFP8 projection is evaluated from the oracle's own quantization of both operands
(oracle.mxfp8.quantize) with float64 accumulation; the bf16 rounding points are those of the
fused GEMM epilogue: y = bf16(acc), bf16(y + bias), bf16(addend + y), bf16(res + bf16(gate y)).

Two modes:
  stage functions (attention_stage, cross_stage, ffn_stage) take the previous stage's hidden
      state, so a GPU run can be checked stage by stage on its own inputs;
  eager_block_fp32 is the plain fp32 torch path (nn.Linear in fp32 on bf16 weights, per-frame
      SDPA, the eager VDA branch), the CPU baseline.

Pins (tests/test_oracle_block.py): LoRA merge against the unmerged sum x W^T + s x A^T B^T;
zero AdaLN gates leave the hidden state of the gated stages unchanged bit for bit; a constant
value in the cross-attention returns that constant; the MXFP8 composition agrees with the
fp32 eager path to MXFP8 accuracy.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch
import torch.nn.functional as F

from . import mxfp8 as _mx
from . import vda as _vda
from . import window as _win


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 values, returned as float64."""
    return x.double().float().to(torch.bfloat16).double()


def _dequantized(x: torch.Tensor) -> torch.Tensor:
    """The MXFP8 value of a [R, K] matrix (oracle quantizer), float32 (exact), cropped to
    [R, K]. Large matrices are processed as independent 1024-row slices on a thread pool;
    128-row-aligned slices quantize exactly as the whole matrix does."""
    r, k = x.shape
    xf = x.float().numpy()

    def one(lo):
        hi = min(r, lo + _SLICE)
        codes, natural = _mx.quantize_natural(xf[lo:hi])
        return _mx.dequant(codes, natural)[:hi - lo, :k].astype(np.float32)

    starts = list(range(0, r, _SLICE))
    if len(starts) == 1:
        return torch.from_numpy(one(0))
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
        return torch.from_numpy(np.concatenate(list(pool.map(one, starts))))


_SLICE = 1024


class QuantizedLinear:
    """An MXFP8 weight (oracle quantizer) kept dequantized, plus its bf16 bias."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        self.n = weight.shape[0]
        self.w = _dequantized(weight)
        self.bias = None if bias is None else bias.double()

    def __call__(self, x, *, addend=None, residual=None, gate=None):
        """x: bf16-valued [R, K] -> the bf16-valued epilogue result (float64 tensor)."""
        y = bf16(_dequantized(x).double() @ self.w.double().T)
        if self.bias is not None:
            y = bf16(y + self.bias)
        if addend is not None:
            y = bf16(addend.double() + y)
        if residual is not None:
            if gate is not None:
                y = bf16(gate.double().reshape(1, -1) * y)
            y = bf16(residual.double() + y)
        return y


def merge_lora(weight, lora_a, lora_b, scale):
    """W + bf16(scale * (B @ A)) per Q/K/V slice (lora.py:80-107: fp32 product, added in the
    weight dtype before MXFP8 conversion). weight [3 * inner, hidden]."""
    inner = weight.shape[0] // 3
    w = weight.clone()
    for i in range(3):
        delta = (lora_b[i].float() @ lora_a[i].float()) * scale
        w[i * inner:(i + 1) * inner] += delta.to(w.dtype)
    return w


class BlockOracle:
    """The block's weights prepared for the oracle. `w` maps names to bf16 CPU tensors (the
    names of the product's random-init weight set); `cfg` supplies hidden, heads, head_dim,
    eps, lora_scale, vda_chunk."""

    def __init__(self, w: dict, cfg):
        self.cfg, self.w = cfg, w
        self.qkv = QuantizedLinear(merge_lora(w["qkv_w"], w["lora_a"], w["lora_b"], cfg.lora_scale),
                                   w["qkv_b"])
        # to_out and to_out_linear as one projection of the concatenated branch outputs:
        # bf16(acc_o + acc_lin) + b_o (one accumulation, then the epilogue's roundings)
        self.o_cat = QuantizedLinear(torch.cat((w["o_w"], w["olin_w"]), dim=1), w["o_b"])
        self.cq = QuantizedLinear(w["cq_w"], w["cq_b"])
        self.ck = QuantizedLinear(w["ck_w"], w["ck_b"])
        self.cv = QuantizedLinear(w["cv_w"], w["cv_b"])
        self.co = QuantizedLinear(w["co_w"], w["co_b"])
        self.up = QuantizedLinear(w["up_w"], w["up_b"])
        self.down = QuantizedLinear(w["down_w"], w["down_b"])

    # ------------------------------------------------------------------ pieces ----
    def tables(self, temb):
        """Six bf16 [1, H] tables: Linear(bf16(SiLU(temb in fp32))) (paper_adaln.py:174-188)."""
        s = bf16(F.silu(temb.float()).double())
        y = bf16(s @ self.w["adaln_w"].double().T + self.w["adaln_b"].double())
        return y.chunk(6, dim=-1)

    def prenorm(self, h, weight, scale, shift):
        t = h.shape[0]
        y = _mx.prenorm(h.float().numpy(), weight.float().numpy(), self.cfg.eps,
                        scale.float().numpy(), shift.float().numpy(), np.zeros(t, np.int64))
        return torch.from_numpy(y).double()

    def small_projections(self, x1, heads=None):
        """softmax gate sigmoid(x Wg^T + b) [T, H]; beta sigmoid(x Wb^T) [T, H]; output gate
        sigmoid(up(down x)) [T, H*D] (attention_gates.py:52-55), bf16 at each torch op.
        `heads` (a list) restricts the three outputs to those heads' columns, in that order;
        each column is computed exactly as in the full projection."""
        w, nh, d = self.w, self.cfg.heads, self.cfg.head_dim
        hs = list(range(nh)) if heads is None else list(heads)
        cols = torch.tensor([i * d + c for i in hs for c in range(d)], dtype=torch.long)
        gw, gb = w["soft_gate_w"][hs], w["soft_gate_b"][hs]
        small = bf16(x1 @ torch.cat((gw, w["beta_w"][hs], w["lgate_down_w"])).double().T)
        n = len(hs)
        # the softmax gate is one Linear with bias (OutputGate.up): bias added before rounding
        soft_gate = bf16(torch.sigmoid(bf16(x1 @ gw.double().T + gb.double())))
        beta = bf16(torch.sigmoid(small[:, n:2 * n]))
        up = bf16(small[:, 2 * n:] @ w["lgate_up_w"][cols].double().T
                  + w["lgate_up_b"][cols].double())
        return soft_gate, beta, bf16(torch.sigmoid(up))

    def out_projection(self, soft, far, h, gate, order="fused"):
        """The attention stage's residual update h + gate * (to_out(soft) + to_out_linear(far)).

        order "fused": one projection of [soft | far] with [W_O | W_Olin], one accumulation:
            bf16(h + bf16(gate * bf16(bf16(acc_O + acc_Olin) + b_O)))   (the product's GEMM)
        order "reference": the reference's two projections, each rounded, then added in bf16
            (hybrid_attention.py:252-254; to_out_linear has no bias, :100-101), then the
            gated residual of _post_ref (fused_block.py:49-51) in bf16:
            o = bf16(bf16(acc_O) + b_O); o = bf16(o + bf16(acc_Olin));
            bf16(h + bf16(gate * o))"""
        if order == "fused":
            return self.o_cat(torch.cat((soft, far), dim=1), residual=h, gate=gate)
        if order != "reference":
            raise ValueError("order must be 'fused' or 'reference'")
        if not hasattr(self, "_o_pair"):
            self._o_pair = (QuantizedLinear(self.w["o_w"], self.w["o_b"]),
                            QuantizedLinear(self.w["olin_w"]))
        o, olin = self._o_pair
        return olin(far, addend=o(soft), residual=h, gate=gate)

    def alpha(self, x1, frames, spatial):
        w, cfg = self.w, self.cfg
        mean = x1.reshape(frames, spatial, -1).float().mean(1)
        return _vda.frame_kda_alpha(mean, w["alpha_down_w"], w["alpha_up_w"], w["dt_bias"],
                                    w["a_log"], cfg.heads, cfg.head_dim)

    # ------------------------------------------------------------------ stages ----
    def attention_stage(self, h, tables, frames, height, width, cos, sin, given=None):
        """h + gate_msa * (O(gated window softmax) + O_lin(VDA)); bf16-valued float64.

        `given` (optional) maps x1, qkv, soft, far to another run's values: each piece is
        still computed here, from the given upstream values where present, so a run can be
        checked piece by piece on its own inputs."""
        cfg, w = self.cfg, self.w
        heads, d, hd = cfg.heads, cfg.head_dim, cfg.heads * cfg.head_dim
        shift, scale, gate = tables[0], tables[1], tables[2]
        spatial = height * width
        t = h.shape[0]
        g = given or {}

        def use(name, own):
            return g[name].double() if name in g else own

        x1 = self.prenorm(h, w["norm1"], scale, shift)
        x1_in = use("x1", x1)
        qkv = self.qkv(x1_in)
        qkv_in = use("qkv", qkv)
        raw_q, raw_k, value = (qkv_in[:, i * hd:(i + 1) * hd].reshape(t, heads, d) for i in range(3))
        soft_gate, beta, lin_gate = self.small_projections(x1_in)
        alpha = self.alpha(x1_in, frames, spatial)
        q = _win.qk_rope(raw_q.to(torch.bfloat16), w["norm_q"], cfg.eps, cos, sin).double()
        k = _win.qk_rope(raw_k.to(torch.bfloat16), w["norm_k"], cfg.eps, cos, sin).double()
        bounds = _vda.window_bounds(frames, cfg.radius)
        mask = _win.dense_mask(t, 0, frames, spatial, bounds)
        o, _ = _win.attention_dense(q, k, value, mask, d ** -0.5)
        soft = _win.softmax_gate(o, soft_gate).double()
        far, _ = _vda.paper_branch(raw_q, raw_k, value, beta, lin_gate.reshape(t, heads, d), alpha,
                                   bounds, frames, spatial, w["vda_norm"].double(), cfg.eps,
                                   chunk_size=cfg.vda_chunk)
        far = bf16(far)
        out = self.out_projection(use("soft", soft), use("far", far), h, gate)
        return out, dict(x1=x1, qkv=qkv, soft=soft, far=far, alpha=alpha)

    def cross_stage(self, h, context, given=None):
        """h + O_c(attention(RMSNorm(norm3(h)) W_q, context W_k, context W_v)); `given` may
        hold another run's co (the attention output) for the last projection."""
        cfg, w = self.cfg, self.w
        heads, d = cfg.heads, cfg.head_dim
        t, L = h.shape[0], context.shape[0]
        zeros = torch.zeros(1, cfg.hidden, dtype=torch.float64)
        x3 = self.prenorm(h, w["norm3"], zeros, zeros)
        q = self.cq(x3).reshape(t, heads, d)
        cx = context.double()
        k = self.ck(cx).reshape(L, heads, d)
        v = self.cv(cx).reshape(L, heads, d)
        q = _win.qk_rope(q.to(torch.bfloat16), w["norm_qc"], cfg.eps).double()
        k = _win.qk_rope(k.to(torch.bfloat16), w["norm_kc"], cfg.eps).double()
        mask = torch.ones(t, L, dtype=torch.bool)
        o, _ = _win.attention_dense(q, k, v, mask, d ** -0.5)
        co = bf16(o.reshape(t, -1))
        co_in = (given or {}).get("co", co).double()
        return self.co(co_in, residual=h), dict(co=co)

    def ffn_stage(self, h, tables, given=None):
        """h + gate_mlp * down(act(up(prenorm(h; norm2, scale_mlp, shift_mlp)))) with act
        GELU-tanh, or SwiGLU a * silu(g) of up = [a | g] (cfg.ffn_act); `given` may hold another
        run's activation as dequantized MXFP8 ("act")."""
        w = self.w
        shift, scale, gate = tables[3], tables[4], tables[5]
        x2 = self.prenorm(h, w["norm2"], scale, shift)
        up = self.up(x2)
        if getattr(self.cfg, "ffn_act", "gelu_tanh") == "swiglu":
            act = torch.from_numpy(_mx.swiglu(up.float().numpy())).double()
        else:
            act = torch.from_numpy(_mx.gelu_tanh(up.float().numpy())).double()
        act_in = (given or {}).get("act", act).double()
        return self.down(act_in, residual=h, gate=gate), dict(up=up, act=act)

    def forward(self, h, temb, context, frames, height, width, cos, sin):
        tables = self.tables(temb)
        h1, _ = self.attention_stage(h.double(), tables, frames, height, width, cos, sin)
        h2, _ = self.cross_stage(h1, context)
        h3, _ = self.ffn_stage(h2, tables)
        return h3, dict(h1=h1, h2=h2, tables=tables)


# ------------------------------------------------------------- eager fp32 (CPU path) ----

def eager_block_fp32(w: dict, cfg, h, temb, context, frames, height, width, cos, sin):
    """The block in fp32 torch on the CPU, as the reference's eager modules evaluate it with
    bf16 weights upcast (no MXFP8): AdaLN tables, RMSNorm/modulation (_pre_ref), nn.Linear
    projections, QK RMSNorm + RoPE, per-frame SDPA (window_softmax_reference), the eager VDA
    branch (branch.py:404-482), gated residuals (_post_ref), cross-attention, GELU-tanh FFN.
    The timed CPU baseline. h [T, H] float; returns float32 [T, H]."""
    f32 = torch.float32
    heads, d, hd, eps = cfg.heads, cfg.head_dim, cfg.heads * cfg.head_dim, cfg.eps
    t, spatial = h.shape[0], height * width
    W = {k: v.to(f32) if v.is_floating_point() else v for k, v in w.items()}
    h = h.to(f32)

    def rms(x, weight):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight

    tables = F.linear(F.silu(temb.to(f32)), W["adaln_w"], W["adaln_b"]).chunk(6, dim=-1)
    shift, scale, gate = tables[:3]
    qkv_w = merge_lora(w["qkv_w"], w["lora_a"], w["lora_b"], cfg.lora_scale).to(f32)
    x1 = rms(h, W["norm1"]) * (1 + scale) + shift
    qkv = F.linear(x1, qkv_w, W["qkv_b"])
    raw_q, raw_k, value = (qkv[:, i * hd:(i + 1) * hd].reshape(t, heads, d) for i in range(3))
    small = F.linear(x1, torch.cat((W["soft_gate_w"], W["beta_w"], W["lgate_down_w"])))
    soft_gate = torch.sigmoid(small[:, :heads] + W["soft_gate_b"])
    beta = torch.sigmoid(small[:, heads:2 * heads])
    lin_gate = torch.sigmoid(F.linear(small[:, 2 * heads:], W["lgate_up_w"], W["lgate_up_b"]))
    mean = x1.reshape(frames, spatial, -1).mean(1)
    alpha = _vda.frame_kda_alpha(mean, W["alpha_down_w"], W["alpha_up_w"], W["dt_bias"],
                                 W["a_log"], heads, d)
    c, s = cos.to(f32)[:, None], sin.to(f32)[:, None]

    def rope(x, weight):
        n = rms(x, weight)
        half = n.shape[-1] // 2
        return n * c + torch.cat((-n[..., half:], n[..., :half]), -1) * s

    q, k = rope(raw_q, W["norm_q"]), rope(raw_k, W["norm_k"])
    bounds = _vda.window_bounds(frames, cfg.radius)
    layout = _Layout(t, frames, spatial)
    o = _win.window_softmax_reference(q, k, value, layout, bounds, d ** -0.5)
    soft = (o * soft_gate[..., None]).reshape(t, hd)
    far = _vda.eager_branch_fp32(raw_q, raw_k, value, beta, lin_gate.reshape(t, heads, d), alpha,
                                 bounds, frames, spatial, W["vda_norm"], eps)
    h = h + gate * (F.linear(soft, W["o_w"], W["o_b"]) + F.linear(far, W["olin_w"]))
    x3 = rms(h, W["norm3"])
    cq = rms(F.linear(x3, W["cq_w"], W["cq_b"]).reshape(t, heads, d), W["norm_qc"])
    ctx = context.to(f32)
    L = ctx.shape[0]
    ck = rms(F.linear(ctx, W["ck_w"], W["ck_b"]).reshape(L, heads, d), W["norm_kc"])
    cv = F.linear(ctx, W["cv_w"], W["cv_b"]).reshape(L, heads, d)
    co = F.scaled_dot_product_attention(cq.transpose(0, 1), ck.transpose(0, 1), cv.transpose(0, 1),
                                        scale=d ** -0.5).transpose(0, 1).reshape(t, hd)
    h = h + F.linear(co, W["co_w"], W["co_b"])
    shift, scale, gate = tables[3:]
    x2 = rms(h, W["norm2"]) * (1 + scale) + shift
    if getattr(cfg, "ffn_act", "gelu_tanh") == "swiglu":
        a, g = F.linear(x2, W["up_w"], W["up_b"]).chunk(2, dim=-1)
        up = a * F.silu(g)
    else:
        up = F.gelu(F.linear(x2, W["up_w"], W["up_b"]), approximate="tanh")
    return h + gate * F.linear(up, W["down_w"], W["down_b"])


class _Layout:
    """The packed geometry window_softmax_reference reads: video rows only."""

    def __init__(self, seq_len, frames, spatial):
        self.seq_len, self.video_start, self.num_frames = seq_len, 0, frames
        self.tokens_per_frame, self.video_end = spatial, frames * spatial

    def global_index(self, device):
        return torch.empty(0, dtype=torch.long, device=device)
