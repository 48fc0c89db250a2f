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


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _bf16(x):
    """Nearest bf16 value(s); a scalar argument gives a Python float."""
    r = omx.bf16_round(np.asarray(x, dtype=np.float64))
    return float(r.reshape(-1)[0]) if np.ndim(x) == 0 else r


def oracle_tables(tensors, cfg, temb):
    """AdaLN tables of the oracle (float64 after each bf16 rounding)."""
    return [t.double() for t in ob.BlockOracle(tensors, cfg).tables(temb)]


def check_adaln_closed_forms(tables_of, w, cfg):
    """AdaLN tables = Linear(bf16(SiLU(temb in fp32))) in the order shift, scale, gate
    (attention), then shift, scale, gate (MLP) (paper_adaln.py:186, 205-212).
    temb = 0 gives SiLU = 0, so every table is its bias; a weight row that is one-hot at
    column j gives bf16(SiLU(temb_j)) at exactly that row's table and position.
    `tables_of(tensors, temb)` returns the six tables as float64 CPU tensors."""
    hd = cfg.hidden
    temb = torch.linspace(-3, 3, hd)[None].to(torch.bfloat16).float()
    tables = tables_of(w.tensors, torch.zeros(1, hd))
    bias = w.adaln_b.double()
    for c in range(6):
        assert torch.equal(tables[c][0], bias[c * hd:(c + 1) * hd]), c
    tensors = dict(w.tensors)
    tensors["adaln_w"] = torch.zeros_like(w.adaln_w)
    tensors["adaln_b"] = torch.zeros_like(w.adaln_b)
    picks = {0: (3, 17), 1: (100, 200), 2: (5, 255), 3: (254, 0), 4: (77, 77), 5: (0, 128)}
    for c, (i, j) in picks.items():
        tensors["adaln_w"][c * hd + i, j] = 1.0
    tables = tables_of(tensors, temb)
    for c, (i, j) in picks.items():
        expect = torch.zeros(hd, dtype=torch.float64)
        expect[i] = _bf16(_bf16(_silu(float(temb[0, j]))))
        assert torch.equal(tables[c][0], expect), c


def test_adaln_tables_closed_forms(small):
    w, _ = small
    check_adaln_closed_forms(lambda t, temb: oracle_tables(t, SMALL, temb), w, SMALL)


def oracle_alpha(tensors, cfg, mean):
    from oracle import vda as ov
    return ov.frame_kda_alpha(mean, tensors["alpha_down_w"], tensors["alpha_up_w"],
                              tensors["dt_bias"], tensors["a_log"], cfg.heads, cfg.head_dim)


def check_alpha_closed_forms(alpha_of, w, cfg):
    """FrameKDAAlpha (layers.py:29-34, 36-69): alpha = exp(-exp(A_log) softplus(up(down(m)) +
    dt_bias)). With zero down/up weights and the fla init dt_bias = dt + log(-expm1(-dt)),
    softplus(dt_bias) = dt exactly, so alpha = exp(-A dt) per head and channel. With
    A_log = 0, dt_bias = 0 and one-hot down/up rows routing frame-mean channel j to output
    (h, c), alpha(h, c) = exp(-softplus(m_j)) = 1 / (1 + e^m_j) and every other channel
    is exp(-softplus(0)) = 1/2. `alpha_of(tensors, mean)` takes per-frame means [F, hidden]
    (bf16 values) and returns alpha [F, heads, head_dim] fp32 on the CPU."""
    nh, d, hd = cfg.heads, cfg.head_dim, cfg.hidden
    g = np.random.default_rng(7)
    a = g.uniform(1, 16, nh)
    dt = np.exp(g.uniform(np.log(1e-3), np.log(1e-1), nh * d))
    tensors = dict(w.tensors)
    tensors["alpha_down_w"] = torch.zeros_like(w.alpha_down_w)
    tensors["alpha_up_w"] = torch.zeros_like(w.alpha_up_w)
    tensors["a_log"] = torch.tensor(np.log(a), dtype=torch.float32)
    tensors["dt_bias"] = torch.tensor(dt + np.log(-np.expm1(-dt)), dtype=torch.float32)
    mean = torch.randn(3, hd, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).float()
    expect = np.exp(-a[:, None] * dt.reshape(nh, d))[None].repeat(3, 0)
    alpha = alpha_of(tensors, mean)
    assert alpha.shape == (3, nh, d) and alpha.dtype == torch.float32
    np.testing.assert_allclose(alpha.numpy(), expect, rtol=3e-6)
    tensors["a_log"] = torch.zeros(nh)
    tensors["dt_bias"] = torch.zeros(nh * d)
    routes = [(11, 4, 1, 127), (200, 9, 0, 0)]      # (mean channel j, latent r, head, channel)
    for j, r, h, c in routes:
        tensors["alpha_down_w"][r, j] = 1.0
        tensors["alpha_up_w"][h * d + c, r] = 1.0
    mean = torch.linspace(-4, 4, 3 * hd).reshape(3, hd).to(torch.bfloat16).float()
    expect = np.full((3, nh, d), 0.5)
    for j, r, h, c in routes:
        expect[:, h, c] = 1.0 / (1.0 + np.exp(mean[:, j].double().numpy()))
    np.testing.assert_allclose(alpha_of(tensors, mean).numpy(), expect, rtol=2e-6)


def test_frame_alpha_closed_forms(small):
    w, _ = small
    check_alpha_closed_forms(lambda t, mean: oracle_alpha(t, SMALL, mean), w, SMALL)


def oracle_gates(tensors, cfg, x1):
    """(soft gate, beta, output gate) of the oracle for x1 [T, hidden] (float64)."""
    return ob.BlockOracle(tensors, cfg).small_projections(x1)


def check_gate_closed_forms(gates_of, w, cfg):
    """The softmax gate sigmoid(x Wg^T + b) per head, beta sigmoid(x Wb^T) and the output
    gate sigmoid(up(down x)) (attention_gates.py:52-55): zero weights give sigmoid(bias)
    (OutputGate's constant init: bias logit(p) gives p), beta 1/2; one-hot rows give
    sigmoid(x_j + b) at exactly the routed head / channel. `gates_of(tensors, x1)` returns
    float64 CPU tensors."""
    nh, d, hd = cfg.heads, cfg.head_dim, cfg.hidden
    tensors = dict(w.tensors)
    for name in ("soft_gate_w", "beta_w", "lgate_down_w", "lgate_up_w"):
        tensors[name] = torch.zeros_like(w.tensors[name])
    logit = lambda p: float(np.log(p / (1 - p)))
    tensors["soft_gate_b"] = torch.full((nh,), logit(0.99)).to(torch.bfloat16)
    tensors["lgate_up_b"] = torch.full((nh * d,), logit(0.9)).to(torch.bfloat16)
    x1 = torch.linspace(-2, 2, 5 * hd).reshape(5, hd).to(torch.bfloat16).double()
    soft, beta, lin = gates_of(tensors, x1)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    assert torch.equal(beta, torch.full((5, nh), 0.5, dtype=torch.float64))
    np.testing.assert_allclose(soft.numpy(), sig(_bf16(logit(0.99))), rtol=2 ** -8)
    np.testing.assert_allclose(lin.numpy(), sig(_bf16(logit(0.9))), rtol=2 ** -8)
    tensors["soft_gate_b"] = torch.zeros(nh, dtype=torch.bfloat16)
    tensors["lgate_up_b"] = torch.zeros(nh * d, dtype=torch.bfloat16)
    tensors["soft_gate_w"][1, 33] = 1.0
    tensors["beta_w"][0, 250] = 1.0
    tensors["lgate_down_w"][7, 3] = 1.0
    tensors["lgate_up_w"][1 * d + 5, 7] = 1.0
    soft, beta, lin = gates_of(tensors, x1)
    xs = x1.numpy()
    np.testing.assert_allclose(soft[:, 1].numpy(), sig(xs[:, 33]), rtol=2 ** -8)
    np.testing.assert_allclose(soft[:, 0].numpy(), 0.5)
    np.testing.assert_allclose(beta[:, 0].numpy(), sig(xs[:, 250]), rtol=2 ** -8)
    np.testing.assert_allclose(lin[:, d + 5].numpy(), sig(xs[:, 3]), rtol=2 ** -8)
    others = np.delete(lin.numpy(), d + 5, axis=1)
    np.testing.assert_allclose(others, 0.5)


def test_gate_projections_closed_forms(small):
    w, _ = small
    check_gate_closed_forms(lambda t, x1: oracle_gates(t, SMALL, x1), w, SMALL)


def test_prenorm_uses_tables_scale_then_shift(small):
    """The first prenorm takes (scale, shift) = tables (1, 0): x_hat (1 + scale) + shift
    (fused_block.py:43-46), checked with a zero-scale / constant-shift table pair."""
    w, orc = small
    h, *_ = inputs(SMALL)
    zero = torch.zeros(1, SMALL.hidden, dtype=torch.float64)
    shift = torch.full((1, SMALL.hidden), 0.25, dtype=torch.float64)
    x = orc.prenorm(h.double(), w.norm1, zero, shift)
    hf = h.double().numpy()
    xhat = hf / np.sqrt((hf ** 2).mean(1, keepdims=True) + SMALL.eps) * w.norm1.double().numpy()
    np.testing.assert_allclose(x.numpy(), _bf16(xhat + 0.25), rtol=2 ** -7, atol=2 ** -9)
    doubled = orc.prenorm(h.double(), w.norm1, torch.ones_like(zero), zero)
    np.testing.assert_allclose(doubled.numpy(), _bf16(2 * xhat), rtol=2 ** -7, atol=2 ** -9)


def test_output_projection_orders_agree_to_one_rounding(small):
    """The fused [O | O_lin] projection (one accumulation) and the reference's order (two
    projections rounded to bf16, then added) differ by bf16 rounding only, well inside
    1e-2 of the update; with to_out_linear's weight zeroed they are identical."""
    w, orc = small
    g = torch.Generator().manual_seed(9)
    inner = SMALL.inner
    soft = torch.randn(64, inner, generator=g).to(torch.bfloat16).double()
    far = torch.randn(64, inner, generator=g).to(torch.bfloat16).double()
    h = torch.randn(64, SMALL.hidden, generator=g).to(torch.bfloat16).double()
    gate = torch.randn(SMALL.hidden, generator=g).to(torch.bfloat16).double()
    fused = orc.out_projection(soft, far, h, gate)
    ref = orc.out_projection(soft, far, h, gate, order="reference")
    assert 0 < float((fused - ref).norm() / (ref - h).norm()) < 1e-2
    tensors = dict(w.tensors)
    tensors["olin_w"] = torch.zeros_like(w.olin_w)
    zo = ob.BlockOracle(tensors, SMALL)
    assert torch.equal(zo.out_projection(soft, far, h, gate),
                       zo.out_projection(soft, far, h, gate, order="reference"))


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
