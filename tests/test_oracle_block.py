"""CPU pins of the block oracle (oracle/block.py) at small widths; no GPU."""
import numpy as np
import pytest
import torch

from oracle import block as ob
from oracle import mxfp8 as omx
from vdn_amd.block import BlockConfig, BlockWeights

SMALL = BlockConfig(hidden=256, heads=2, head_dim=128, ffn=384, context=16, lora_rank=8,
                    lora_scale=0.5)
FRAMES, HEIGHT, WIDTH = 4, 4, 4


def inputs(cfg, seed=3):
    g = torch.Generator().manual_seed(seed)
    t = FRAMES * HEIGHT * WIDTH
    h = torch.randn(t, cfg.hidden, generator=g).to(torch.bfloat16)
    temb = torch.randn(1, cfg.hidden, generator=g)
    ctx = torch.randn(cfg.context, cfg.hidden, generator=g).to(torch.bfloat16)
    cos, sin = ob._win.rope_tables_3d(FRAMES, HEIGHT, WIDTH)
    return h, temb, ctx, cos, sin


@pytest.fixture(scope="module")
def small():
    w = BlockWeights.random(SMALL, seed=5)
    return w, ob.BlockOracle(w.tensors, SMALL)


def test_lora_merge_matches_the_unmerged_sum():
    g = torch.Generator().manual_seed(0)
    hd, r = 64, 4
    w = (torch.randn(3 * hd, hd, generator=g) * 0.02).to(torch.bfloat16)
    a = (torch.randn(3, r, hd, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(3, hd, r, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(5, hd, generator=g, dtype=torch.float64)
    merged = ob.merge_lora(w, a, b, 0.75).double()
    unmerged = torch.cat([x @ w[i * hd:(i + 1) * hd].double().T
                          + 0.75 * (x @ a[i].double().T) @ b[i].double().T for i in range(3)], 1)
    # each merged element differs from the exact sum by one bf16 rounding of the sum
    bound = x.abs() @ torch.from_numpy(omx.bf16_ulp(merged.numpy()) / 2 + 1e-12).T * 1.01
    assert torch.all((x @ merged.T - unmerged).abs() <= bound + 1e-9)
    # a dropped scale or a transposed product would be far outside that bound
    wrong = ob.merge_lora(w, a, b, 1.0).double()
    assert not torch.all((x @ wrong.T - unmerged).abs() <= bound + 1e-9)


def test_zero_gate_tables_make_the_gated_stages_identities(small):
    w, orc = small
    h, temb, ctx, cos, sin = inputs(SMALL)
    tables = list(orc.tables(temb))
    hd = h.double()
    for gate_index, stage in ((2, "attention"), (5, "ffn")):
        zeroed = list(tables)
        zeroed[gate_index] = torch.zeros_like(tables[gate_index])
        if stage == "attention":
            out, _ = orc.attention_stage(hd, zeroed, FRAMES, HEIGHT, WIDTH, cos, sin)
        else:
            out, _ = orc.ffn_stage(hd, zeroed)
        assert torch.equal(out, hd), stage
        # with the real gate the stage changes the state
        if stage == "attention":
            live, _ = orc.attention_stage(hd, tables, FRAMES, HEIGHT, WIDTH, cos, sin)
        else:
            live, _ = orc.ffn_stage(hd, tables)
        assert (live - hd).abs().max() > 1e-2, stage


def test_table_order_shift_scale_gate(small):
    """Tables are (shift, scale, gate) x (attention, mlp): the first prenorm uses tables 0/1."""
    w, orc = small
    h, temb, *_ = inputs(SMALL)
    t = orc.tables(temb)
    x = orc.prenorm(h.double(), w.norm1, t[1], t[0])
    f = np.float32
    hf = h.float().numpy()
    inv = 1 / np.sqrt((hf.astype(np.float64) ** 2).mean(1, keepdims=True) + SMALL.eps)
    expect = (hf * inv) * w.norm1.float().numpy() * (1 + t[1].numpy()) + t[0].numpy()
    assert np.allclose(x.numpy(), expect, rtol=2 ** -7, atol=2 ** -7)
    assert t[0].shape == (1, SMALL.hidden) and len(t) == 6


def test_constant_context_value_passes_through_cross_attention(small):
    w, _ = small
    tensors = dict(w.tensors)
    tensors["cv_w"] = torch.zeros_like(tensors["cv_w"])
    c = torch.linspace(-1, 1, SMALL.hidden).to(torch.bfloat16)
    tensors["cv_b"] = c
    orc = ob.BlockOracle(tensors, SMALL)
    h, _, ctx, *_ = inputs(SMALL)
    out, parts = orc.cross_stage(h.double(), ctx)
    # every query's attention output is the constant value row, whatever the scores
    assert torch.allclose(parts["co"], c.double().expand_as(parts["co"]), atol=0, rtol=2 ** -8)


def test_mxfp8_composition_tracks_the_fp32_eager_block(small):
    """The oracle's MXFP8 block and the plain fp32 block agree to MXFP8 accuracy (E4M3 has
    3 mantissa bits: a few percent per projection), per stage delta and end to end."""
    w, orc = small
    h, temb, ctx, cos, sin = inputs(SMALL)
    out, parts = orc.forward(h, temb, ctx, FRAMES, HEIGHT, WIDTH, cos, sin)
    eager = ob.eager_block_fp32(w.tensors, SMALL, h, temb, ctx, FRAMES, HEIGHT, WIDTH, cos, sin)
    delta, ref = out - h.double(), eager.double() - h.double()
    rel = (delta - ref).norm() / ref.norm()
    assert rel < 0.12, rel
    # a block with the FFN (its smallest stage here) dropped is well outside that bound
    no_ffn = parts["h2"] - h.double()
    assert (no_ffn - ref).norm() / ref.norm() > 0.2


SWIGLU = BlockConfig(hidden=384, heads=2, head_dim=128, ffn=320, ffn_act="swiglu", context=16,
                     lora_rank=8, lora_scale=0.5)


def test_swiglu_block_with_attention_width_unlike_hidden():
    """VDN-H3's structure at small widths (hidden 384, attention 2 x 128, SwiGLU FFN 320):
    the MXFP8 composition tracks the fp32 eager block, the activation is a * silu(g) of the up
    projection's halves [a | g], and swapping the halves is far outside the bound."""
    w = BlockWeights.random(SWIGLU, seed=6)
    orc = ob.BlockOracle(w.tensors, SWIGLU)
    assert w.qkv_w.shape == (3 * 256, 384) and w.o_w.shape == (384, 256)
    assert w.up_w.shape == (640, 384) and w.down_w.shape == (384, 320)
    h, temb, ctx, cos, sin = inputs(SWIGLU)
    out, parts = orc.forward(h, temb, ctx, FRAMES, HEIGHT, WIDTH, cos, sin)
    eager = ob.eager_block_fp32(w.tensors, SWIGLU, h, temb, ctx, FRAMES, HEIGHT, WIDTH, cos, sin)
    delta, ref = out - h.double(), eager.double() - h.double()
    assert (delta - ref).norm() / ref.norm() < 0.12
    h3, own = orc.ffn_stage(parts["h2"], parts["tables"])
    up = own["up"]
    a, g = up[:, :320], up[:, 320:]
    expect = omx.bf16_round((a * g / (1 + torch.exp(-g))).numpy())
    assert np.allclose(own["act"].numpy(), expect, rtol=2 ** -7, atol=1e-6)
    swapped = omx.bf16_round((g * a / (1 + torch.exp(-a))).numpy())
    assert not np.allclose(own["act"].numpy(), swapped, rtol=2 ** -7, atol=1e-6)
