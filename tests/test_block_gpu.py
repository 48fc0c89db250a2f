"""Hybrid DiT block on the GPU against the block oracle: piece by piece on the run's own
inputs, and end to end. Widths: a small block and the full 5120-wide block (40 x 128 heads,
FFN 13824, 512 context rows) on a short clip. Tolerance: relative L2 <= 1e-2 on every
projection, attention output and residual-stage delta computed from the run's own inputs;
5e-2 on the free-running block delta (MXFP8 rounding-boundary noise, see check())."""
import pytest
import torch

from oracle import block as ob
from oracle import mxfp8 as omx
from oracle import window as ow
from vdn_amd import window as vw
from vdn_amd.block import (BlockConfig, BlockWeights, FinitePredicate, HybridDiTBlock,
                           cross_attention_plan, make_inputs)

pytestmark = pytest.mark.gpu

SMALL = BlockConfig(hidden=256, heads=2, head_dim=128, ffn=384, context=16, lora_rank=8,
                    lora_scale=0.5)
WIDE = BlockConfig()
# VDN-H3's widths: hidden 5376, 56 x 128 heads (attention width 7168), SwiGLU FFN 14336
# (up 5376 -> 28672 = [a | g]); and a small block with the same structure
H3 = BlockConfig(hidden=5376, heads=56, head_dim=128, ffn=14336, ffn_act="swiglu")
SMALL_H3 = BlockConfig(hidden=384, heads=2, head_dim=128, ffn=320, ffn_act="swiglu", context=16,
                       lora_rank=8, lora_scale=0.5)
# an odd head count (the gate projection runs one zero-padded extra head)
ODD_HEADS = BlockConfig(hidden=320, heads=5, head_dim=128, ffn=384, context=16, lora_rank=8,
                        lora_scale=0.5)
REL = 1e-2
END_TO_END = 5e-2


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def run(cfg, frames, height, width, seed):
    torch.manual_seed(seed)
    w = BlockWeights.random(cfg, seed, device="cuda")
    block = HybridDiTBlock(cfg, w)
    hidden, temb, ctx, layout, (cos, sin) = make_inputs(cfg, frames, height, width, seed + 1,
                                                       device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(frames, cfg.radius),
                                        device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")
    out, parts = block(hidden, temb, ctx, layout, (cos, sin), plan, cplan, return_parts=True)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in w.tensors.items()}
    oracle = ob.BlockOracle(cpu, cfg)
    parts = {k: (tuple(x.cpu() for x in v) if isinstance(v, tuple) else v.cpu())
             for k, v in parts.items()}
    return dict(cfg=cfg, oracle=oracle, hidden=hidden.cpu(), temb=temb.cpu(), ctx=ctx.cpu(),
                cos=cos.cpu(), sin=sin.cpu(), out=out.cpu(), parts=parts,
                geometry=(frames, height, width))


def ffn_activation(codes_scales, rows, n):
    """Dequantized FFN activation from the fused producer's MXFP8 codes and scales."""
    codes, flat = (t.numpy() for t in codes_scales)
    rp, kp = codes.shape
    natural = omx.unswizzle(flat, rp, kp)
    return torch.from_numpy(omx.dequant(codes, natural)[:rows, :n])


def mxfp8_value(x):
    """The MXFP8 value (oracle quantizer, dequantized) of a bf16-valued matrix."""
    codes, natural, _ = omx.quantize(x.float().numpy())
    return torch.from_numpy(omx.dequant(codes, natural)[:x.shape[0], :x.shape[1]])


def check(r):
    cfg, orc, p = r["cfg"], r["oracle"], r["parts"]
    frames, height, width = r["geometry"]
    h0 = r["hidden"].double()
    tables = orc.tables(r["temb"])
    for mine, theirs in zip(p["tables"], tables):
        assert rel_l2(mine, theirs) < 4e-3
    gpu_tables = tuple(t.double() for t in p["tables"])
    given = {k: p[k] for k in ("x1", "qkv", "soft", "far")}
    h1, own = orc.attention_stage(h0, gpu_tables, frames, height, width, r["cos"], r["sin"],
                                  given=given)
    errors = {name: rel_l2(p[name], own[name]) for name in ("x1", "qkv", "soft", "far")}
    errors["h1 delta"] = rel_l2(p["h1"].double() - h0, h1 - h0)
    h1g = p["h1"].double()
    h2, own = orc.cross_stage(h1g, r["ctx"], given={"co": p["co"]})
    errors["co"] = rel_l2(p["co"], own["co"])
    errors["h2 delta"] = rel_l2(p["h2"].double() - h1g, h2 - h1g)
    h2g = p["h2"].double()
    act = ffn_activation(p["ffn_codes"], r["hidden"].shape[0], cfg.ffn)
    h3, own = orc.ffn_stage(h2g, gpu_tables, given={"act": act})
    errors["act"] = rel_l2(act, mxfp8_value(own["act"]))
    errors["h3 delta"] = rel_l2(r["out"].double() - h2g, h3 - h2g)
    print({k: f"{v:.2e}" for k, v in errors.items()}, flush=True)
    bad = {k: v for k, v in errors.items() if not v < REL}
    assert not bad, bad
    # End to end from the oracle's own tables and stages. Free-running, a one-ulp bf16
    # difference upstream can move a value across an E4M3 rounding boundary (3 mantissa bits,
    # a 1/16 step) in every later quantization, so the bound is the MXFP8 noise floor: well
    # under the ~8% by which the MXFP8 block itself differs from the fp32 block.
    free, fparts = orc.forward(r["hidden"], r["temb"], r["ctx"], frames, height, width, r["cos"],
                               r["sin"])
    end = {"h1": rel_l2(p["h1"].double() - h0, fparts["h1"] - h0),
           "out": rel_l2(r["out"].double() - h0, free - h0)}
    print(f"end-to-end block delta rel-L2 {end}", flush=True)
    assert end["out"] < END_TO_END


def test_small_block_matches_oracle():
    check(run(SMALL, 4, 4, 8, seed=11))


def test_odd_head_count_block_matches_oracle():
    check(run(ODD_HEADS, 4, 4, 8, seed=13))


def test_full_width_block_short_clip_matches_oracle():
    check(run(WIDE, 4, 4, 8, seed=12))


def test_small_swiglu_block_with_attention_width_unlike_hidden_matches_oracle():
    check(run(SMALL_H3, 4, 4, 8, seed=21))


def test_h3_width_block_short_clip_matches_oracle():
    check(run(H3, 3, 4, 8, seed=22))


def test_block_is_deterministic_and_leaves_its_input_alone():
    cfg = SMALL
    w = BlockWeights.random(cfg, 3, device="cuda")
    block = HybridDiTBlock(cfg, w)
    hidden, temb, ctx, layout, rope = make_inputs(cfg, 3, 5, 7, 4, device="cuda")
    keep = hidden.clone()
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(3, 1), device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")
    a = block(hidden, temb, ctx, layout, rope, plan, cplan)
    b = block(hidden, temb, ctx, layout, rope, plan, cplan)
    torch.cuda.synchronize()
    assert torch.equal(hidden, keep)
    assert torch.equal(a, b), "the block is deterministic run to run"
    assert torch.isfinite(a.float()).all()


def test_side_stream_schedule_matches_serial_over_chained_blocks():
    """The overlapped schedule (gate projection, VDA branch and context projections on a side
    stream) and the serial one give the same bytes over four chained blocks launched back to
    back with no host sync between them, so the caching allocator hands memory freed on one
    stream to the other while earlier blocks are still running."""
    cfg = WIDE
    w = BlockWeights.random(cfg, 7, device="cuda")
    block = HybridDiTBlock(cfg, w)
    hidden, temb, ctx, layout, rope = make_inputs(cfg, 3, 4, 8, 6, device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(3, 1), device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")

    def chain(overlap):
        block.overlap_vda = overlap
        h = hidden
        for _ in range(4):
            h = block(h, temb, ctx, layout, rope, plan, cplan)
        torch.cuda.synchronize()
        return h

    try:
        with torch.no_grad():
            first, serial, again = chain(True), chain(False), chain(True)
    finally:
        block.overlap_vda = True
    assert torch.equal(first, serial)
    assert torch.equal(first, again)
    assert torch.isfinite(first.float()).all()


def test_fused_mxfp8_epilogues_give_the_unfused_block():
    """The block's default path quantizes the attention, VDA and cross-attention outputs in
    their kernels; return_parts keeps them in bf16 and quantizes them separately. Both feed
    the same bytes to the output projections, so the outputs are identical."""
    cfg = WIDE
    w = BlockWeights.random(cfg, 5, device="cuda")
    block = HybridDiTBlock(cfg, w)
    hidden, temb, ctx, layout, rope = make_inputs(cfg, 3, 4, 8, 6, device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(3, 1), device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")
    with torch.no_grad():
        fused = block(hidden, temb, ctx, layout, rope, plan, cplan)
        unfused, _ = block(hidden, temb, ctx, layout, rope, plan, cplan, return_parts=True)
    assert torch.equal(fused, unfused)


def test_rope_tables_match_the_oracle_restatement():
    cos, sin = vw.rope_tables_3d(3, 5, 7, device="cuda", dtype=torch.float32)
    oc, os_ = ow.rope_tables_3d(3, 5, 7)
    assert torch.allclose(cos.cpu().double(), oc, atol=1e-6)
    assert torch.allclose(sin.cpu().double(), os_, atol=1e-6)


@torch.no_grad()
@pytest.mark.parametrize("w_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows", [300, 1037])
def test_cross_attention_query_norm_in_kernel_equals_norm_pass(w_dtype, rows):
    """The queries' RMSNorm fused into the MXFP8-output attention gives the same codes and
    scales as qk_rmsnorm followed by the attention (partial last query blocks included)."""
    from vdn_amd import mxfp8 as vm
    from vdn_amd.block import cross_attention
    g = torch.Generator().manual_seed(rows)
    heads, d, ctx = 3, 128, 77
    q = (torch.randn(rows, heads, d, generator=g) * 3).bfloat16().cuda()
    k = torch.randn(ctx, heads, d, generator=g).bfloat16().cuda()
    v = torch.randn(ctx, heads, d, generator=g).bfloat16().cuda()
    w = (torch.rand(d, generator=g) + 0.5).to(w_dtype).cuda()
    plan = cross_attention_plan(rows, ctx, "cuda")
    qa, sa = vm.empty_activation(rows, heads * d, "cuda")
    qb, sb = vm.empty_activation(rows, heads * d, "cuda")
    cross_attention(q, k, v, plan, d ** -0.5, out_mxfp8=(qa, sa, 0), q_norm=(w, 1e-6))
    cross_attention(vw.qk_rmsnorm(q, w, 1e-6), k, v, plan, d ** -0.5, out_mxfp8=(qb, sb, 0))
    torch.cuda.synchronize()
    assert torch.equal(qa, qb) and torch.equal(sa, sb)
    with pytest.raises(ValueError, match="MXFP8-output form"):
        cross_attention(q, k, v, plan, d ** -0.5, q_norm=(w, 1e-6))


def test_guard_receives_device_predicates():
    """guard= hands the three prenorm producers' row flags and the projections' flag to
    guard.predicate as device bool tensors (paper_block_forward, fused_block.py:144-155) and
    leaves the output unchanged; a NaN in the hidden state and an inf in the context each
    make the predicate false."""
    cfg = SMALL
    w = BlockWeights.random(cfg, 31, device="cuda")
    block = HybridDiTBlock(cfg, w)
    hidden, temb, ctx, layout, rope = make_inputs(cfg, 4, 4, 8, 32, device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(4, cfg.radius), device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")

    class Recorder(FinitePredicate):
        def __init__(self):
            super().__init__("cuda")
            self.seen = []

        def predicate(self, parts):
            self.seen.append((parts.device.type, parts.dtype))
            super().predicate(parts)

    guard = Recorder()
    out = block(hidden, temb, ctx, layout, rope, plan, cplan, guard=guard)
    ref = block(hidden, temb, ctx, layout, rope, plan, cplan)
    assert torch.equal(out, ref)
    assert guard.seen == [("cuda", torch.bool)] * 4
    guard.check("block")
    bad = hidden.clone()
    bad[7, 3] = float("nan")
    block(bad, temb, ctx, layout, rope, plan, cplan, guard=guard)
    with pytest.raises(FloatingPointError):
        guard.check("block")
    bad_ctx = ctx.clone()
    bad_ctx[2, 5] = float("inf")
    block(hidden, temb, bad_ctx, layout, rope, plan, cplan, guard=guard)
    with pytest.raises(FloatingPointError):
        guard.check("block")
    block(hidden, temb, ctx, layout, rope, plan, cplan, guard=guard)
    guard.check("block")
