"""GPU parity of the window attention and QK norm/RoPE kernels against the oracle, at the
reference tests' tolerances (tests/test_paper_stack_attention_window.py:121-212,
tests/test_paper_stack_attention_rope.py:466-525)."""
import pytest
import torch

from oracle import window as ow
from vdn_amd import window as vw

pytestmark = pytest.mark.gpu

LAYOUTS = [(0, 0), (3, 0), (0, 4), (3, 4)]
GEOMETRY = [(1, 0, 0), (2, 5, 1), (7, 3, 0), (7, 3, 1), (7, 0, 1), (7, 5, 1), (7, 0, 99)]


@pytest.mark.parametrize("before,after", LAYOUTS)
@pytest.mark.parametrize("frames,chunk,radius", GEOMETRY)
@pytest.mark.parametrize("anchor", ["none", "rows", "columns", "both"])
@torch.no_grad()
def test_dense_fp32_oracle(device, before, after, frames, chunk, radius, anchor):
    torch.manual_seed(819)
    layout = vw.SequenceLayout(before + frames * 3 + after, before, frames, 3)
    bounds = vw.window_bounds(frames, radius, chunk)
    backing = torch.randn(layout.seq_len + 5, 3, 14, 128, device=device, dtype=torch.bfloat16)
    q, k, v = [backing[:, i, 3:10] for i in range(3)]
    old = backing.clone()
    plan = vw.prepare_paper_window_plan(layout, bounds, anchor, device=device, max_query_rows=5,
                                        max_gather_rows=2 * layout.seq_len)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    s = layout.seq_len
    mask = ow.dense_mask(s, before, frames, 3, bounds, anchor)
    expected, el = ow.attention_dense(q[:s].cpu(), k[:s].cpu(), v[:s].cpu(), mask, 128 ** -.5)
    got = out[:s].float().cpu()
    torch.testing.assert_close(got, expected, atol=.009, rtol=.015)
    assert ((got - expected).norm() / expected.norm()) < .004
    torch.testing.assert_close(lse[:s].cpu(), el, atol=3e-5, rtol=3e-6)
    assert out[s:].count_nonzero() == 0
    assert torch.isneginf(lse[s:]).all()
    assert torch.equal(backing, old)
    assert out.is_contiguous() and out.data_ptr() != backing.data_ptr()


@pytest.mark.parametrize("growth", [1.0, -1.0])
@torch.no_grad()
def test_large_scores_lazy_rescale(device, growth):
    """Scores of up to several hundred (log2 units) whose per-tile maximum grows (or shrinks)
    from one key tile to the next: the running maximum is raised many times past the lazy
    threshold (8) and every raise rescales the accumulators. Dense fp32 oracle at the
    reference test's tolerances; the log-sum-exp at a tolerance relative to its size."""
    torch.manual_seed(77)
    frames, spatial = 3, 300
    layout = vw.SequenceLayout(frames * spatial, 0, frames, spatial)
    bounds = vw.window_bounds(frames, 1)
    n = layout.seq_len
    q = torch.randn(n, 2, 128) * 8
    # key magnitude ramps over the sequence, so each 128-key tile's maximum differs from the
    # previous one by far more than the threshold
    ramp = torch.linspace(1.0, 6.0, n)
    if growth < 0:
        ramp = ramp.flip(0)
    k = torch.randn(n, 2, 128) * ramp[:, None, None]
    v = torch.randn(n, 2, 128)
    q, k, v = (t.to(device=device, dtype=torch.bfloat16) for t in (q, k, v))
    plan = vw.prepare_paper_window_plan(layout, bounds, device=device)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    mask = ow.dense_mask(n, 0, frames, spatial, bounds, "none")
    expected, el = ow.attention_dense(q.cpu(), k.cpu(), v.cpu(), mask, 128 ** -.5)
    assert el.abs().max() > 100, "the scores must span far more than the lazy threshold"
    got = out.float().cpu()
    assert torch.isfinite(got).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(got, expected, atol=.009, rtol=.015)
    torch.testing.assert_close(lse.cpu(), el, atol=3e-5, rtol=3e-6)


@pytest.mark.parametrize("spatial", [300, 470])
@torch.no_grad()
def test_partial_last_query_block(device, spatial):
    """Frames of 300 and 470 tokens end in a 44- and a 214-row query block: some waves of that
    block hold queries, the rest hold none and only stage tiles. Dense fp32 oracle."""
    torch.manual_seed(31)
    frames = 3
    layout = vw.SequenceLayout(frames * spatial, 0, frames, spatial)
    bounds = vw.window_bounds(frames, 1)
    q, k, v = [torch.randn(layout.seq_len, 2, 128, device=device, dtype=torch.bfloat16)
               for _ in range(3)]
    plan = vw.prepare_paper_window_plan(layout, bounds, device=device)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    mask = ow.dense_mask(layout.seq_len, 0, frames, spatial, bounds, "none")
    expected, el = ow.attention_dense(q.cpu(), k.cpu(), v.cpu(), mask, 128 ** -.5)
    torch.testing.assert_close(out.float().cpu(), expected, atol=.009, rtol=.015)
    torch.testing.assert_close(lse.cpu(), el, atol=3e-5, rtol=3e-6)


@torch.no_grad()
def test_constant_values_anchor_union_mass(device):
    layout = vw.SequenceLayout(45, 2, 13, 3)
    bounds = vw.window_bounds(13, 1, 3)
    q = torch.zeros(45, 7, 128, device=device, dtype=torch.bfloat16)
    v = torch.arange(45, device=device, dtype=torch.float32)[:, None, None].expand_as(q).to(q.dtype)
    p = vw.prepare_paper_window_plan(layout, bounds, "columns", device=device, max_gather_rows=70)
    out, lse = vw.paper_window_attention(q, q, v, p, enabled=True, return_lse=True)
    mask = ow.dense_mask(45, 2, 13, 3, bounds, "columns")
    expected = (mask.float() @ torch.arange(45).float()) / mask.sum(-1)
    torch.testing.assert_close(out[:, 0, 0].cpu(), expected.bfloat16(), rtol=0, atol=0)
    torch.testing.assert_close(lse[:, 0].cpu(), mask.sum(-1).float().log(), rtol=1e-6, atol=1e-6)


@torch.no_grad()
def test_global_only_and_custom_stream(device):
    layout = vw.SequenceLayout(13, 7, 0, 1)
    plan = vw.prepare_paper_window_plan(layout, [], device=device, max_gather_rows=1, max_query_rows=4)
    q, k, v = [torch.randn(15, 7, 128, device=device, dtype=torch.bfloat16) for _ in range(3)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        out = vw.paper_window_attention(q, k, v, plan, enabled=True)
    torch.cuda.current_stream().wait_stream(stream)
    expected, _ = ow.attention_dense(q[:13].cpu(), k[:13].cpu(), v[:13].cpu(),
                                     torch.ones(13, 13, dtype=torch.bool), 128 ** -.5)
    torch.testing.assert_close(out[:13].float().cpu(), expected, rtol=.015, atol=.009)
    assert out[13:].count_nonzero() == 0


@torch.no_grad()
def test_reject_bad_runtime_contract(device):
    p = vw.prepare_paper_window_plan(vw.SequenceLayout(7, 1, 2, 3), [(0, 1)] * 2, device=device)
    q = torch.randn(7, 7, 128, device=device, dtype=torch.bfloat16)
    for args in ((q[:6],) * 3, (q, q, q[:6]), (q.float(),) * 3, (q[..., ::2],) * 3):
        with pytest.raises(ValueError):
            vw.paper_window_attention(*args, p, enabled=True)
    with pytest.raises(ValueError, match="finite"):
        vw.paper_window_attention(q, q, q, p, scale=float("nan"), enabled=True)
    cp = vw.prepare_paper_window_plan(p.layout, p.bounds)
    with pytest.raises(ValueError, match="same CUDA"):
        vw.paper_window_attention(q, q, q, cp, enabled=True)


@torch.no_grad()
def test_fused_gate_equals_separate_gate(device):
    torch.manual_seed(3)
    layout = vw.SequenceLayout(4 * 300, 0, 4, 300)
    bounds = vw.window_bounds(4, 1)
    q, k, v = [torch.randn(1200, 5, 128, device=device, dtype=torch.bfloat16) for _ in range(3)]
    gate = torch.rand(1200, 5, 1, device=device, dtype=torch.bfloat16)
    plan = vw.prepare_paper_window_plan(layout, bounds, device=device)
    plain = vw.paper_window_attention(q, k, v, plan, enabled=True)
    fused = vw.paper_window_attention(q, k, v, plan, enabled=True, gate=gate)
    assert torch.equal(fused.reshape(1200, -1), vw.apply_softmax_gate(plain, gate))


@torch.no_grad()
def test_c4_full_shape_sampled(device):
    """C4: 108,000 tokens (30 frames x 3600), 40 heads, d 128, +-1-frame window. Sampled
    queries (every frame edge and interior, several heads) against the fp32 oracle."""
    frames, spatial, h = 30, 3600, 40
    n = frames * spatial
    g = torch.Generator().manual_seed(4)
    q, k, v = [(torch.randn(n, h, 128, generator=g) / 128 ** .5).to(torch.bfloat16) for _ in range(3)]
    layout = vw.SequenceLayout(n, 0, frames, spatial)
    bounds = vw.window_bounds(frames, 1)
    plan = vw.prepare_paper_window_plan(layout, bounds, device=device)
    out, lse = vw.paper_window_attention(q.to(device), k.to(device), v.to(device), plan,
                                         enabled=True, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    for f in (0, 1, 14, 29):
        lo, hi = max(0, f - 1), min(frames - 1, f + 1)
        keys = slice(lo * spatial, (hi + 1) * spatial)
        rows = torch.cat([torch.arange(f * spatial, f * spatial + 130),
                          torch.arange((f + 1) * spatial - 20, (f + 1) * spatial)])
        for hh in (0, 17, 39):
            qs = q[rows, hh].float()
            scores = qs @ k[keys, hh].float().T * 128 ** -.5
            ref = scores.softmax(-1) @ v[keys, hh].float()
            torch.testing.assert_close(out[rows, hh].float(), ref, atol=.009, rtol=.015)
            torch.testing.assert_close(lse[rows, hh], scores.logsumexp(-1), atol=3e-5, rtol=3e-6)


# ------------------------------------------------------------------------------ RoPE ----

def rope_inputs(d=128, r=96, layout="qkv", t=13):
    g = torch.Generator().manual_seed(194)
    h = 7
    if layout == "qkv":
        storage = torch.randn(t, 3 * h * d, generator=g).bfloat16()
        q = storage[:, :h * d].view(t, h, d)
        k = storage[:, h * d:2 * h * d].view(t, h, d)
    else:
        storage = torch.randn(t, 3, h * 2, d * 2, generator=g).bfloat16()
        q, k = storage[:, 0, ::2, ::2], storage[:, 1, ::2, ::2]
    qw = (torch.rand(d * 2, generator=g) + 0.5).bfloat16()[::2]
    kw = (torch.rand(d * 2, generator=g) + 0.5).bfloat16()[::2]
    angles = torch.randn(t, r * 2, generator=g)
    return storage, q, k, qw, kw, angles.cos()[:, ::2], angles.sin()[:, ::2]


@pytest.mark.parametrize("layout", ["qkv", "inner"])
@pytest.mark.parametrize("r", [None, 96, 128])
@torch.no_grad()
def test_rope_independent_oracle_strided_inputs(device, layout, r):
    storage, q, k, qw, kw, c, s = rope_inputs(r=r or 96, layout=layout, t=33)
    backing = storage.to(device)
    qg = backing.as_strided(q.shape, q.stride(), q.storage_offset())
    kg = backing.as_strided(k.shape, k.stride(), k.storage_offset())
    qwd, kwd = qw.to(device), kw.to(device)
    cg, sg = (None, None) if r is None else (c.to(device), s.to(device))
    before = backing.clone()
    outputs = vw.paper_qk_rmsnorm_rope(qg, kg, qwd, kwd, 1e-5, cg, sg, enabled=True)
    for output, raw, weight in zip(outputs, (q, k), (qw, kw)):
        expected = ow.qk_rope(raw, weight, 1e-5, None if r is None else c, None if r is None else s)
        err = (output.float().cpu() - expected.float()).norm() / expected.float().norm()
        assert err.item() < 2e-3
        torch.testing.assert_close(output.cpu(), expected, rtol=0.02, atol=.032)
        assert output.is_contiguous() and output.shape == (33, 7, 128)
    assert torch.equal(backing, before)
    assert outputs[0].data_ptr() != outputs[1].data_ptr()


@pytest.mark.parametrize("heads,tables", [(7, torch.float32), (40, torch.bfloat16),
                                          (2, torch.bfloat16)])
@torch.no_grad()
def test_rope_full_width_fast_form_matches_general_form(device, heads, tables):
    """D = R = 128 on 16-byte rows takes the per-token fast form; the same values behind a
    channel stride of 2 take the general per-row form. Both round the same way, so their
    outputs are bit-identical (head counts below, at and above a multiple of 4)."""
    g = torch.Generator().manual_seed(heads)
    t = 37
    storage = (torch.randn(t, 3 * heads * 128, generator=g) * 3).bfloat16()
    q = storage[:, :heads * 128].view(t, heads, 128)
    k = storage[:, heads * 128:2 * heads * 128].view(t, heads, 128)
    qw = (torch.rand(128, generator=g) + 0.5).bfloat16()
    kw = (torch.rand(128, generator=g) + 0.5).float()
    angles = torch.randn(t, 128, generator=g) * 4
    c, s = angles.cos().to(tables), angles.sin().to(tables)
    args = (qw.to(device), kw.to(device), 1e-6, c.to(device), s.to(device))
    fast = vw.paper_qk_rmsnorm_rope(q.to(device), k.to(device), *args, enabled=True)
    wide = torch.zeros(t, heads, 256, dtype=torch.bfloat16)
    wide2 = torch.zeros(t, heads, 256, dtype=torch.bfloat16)
    wide[:, :, ::2], wide2[:, :, ::2] = q, k
    general = vw.paper_qk_rmsnorm_rope(wide.to(device)[:, :, ::2], wide2.to(device)[:, :, ::2],
                                       *args, enabled=True)
    for a, b, raw, w in zip(fast, general, (q, k), (qw, kw)):
        assert torch.equal(a, b)
        torch.testing.assert_close(a.cpu(), ow.qk_rope(raw, w, 1e-6, c.float(), s.float()),
                                   atol=.032, rtol=.02)


@torch.no_grad()
def test_rope_bf16_intermediate_round_trap(device):
    g = torch.Generator().manual_seed(715)
    x = torch.ones(3, 7, 128, dtype=torch.bfloat16)
    w = (torch.rand(128, generator=g) * 1.7 + .1).bfloat16()
    angles = torch.randn(3, 96, generator=g)
    c, s = angles.cos(), angles.sin()
    expected = ow.qk_rope(x, w, .25, c, s)
    assert torch.count_nonzero(expected != ow.qk_rope(x, w, .25, c, s, round_norm=False)) > 100
    xd = x.to(device)
    out, _ = vw.paper_qk_rmsnorm_rope(xd, xd, w.to(device), w.to(device), .25, c.to(device),
                                      s.to(device), enabled=True)
    torch.testing.assert_close(out.cpu(), expected, rtol=0, atol=0)


@pytest.mark.parametrize("d,r", [(64, 32), (256, 192)])
@torch.no_grad()
def test_rope_other_widths_fp32_weights_strided_tables(device, d, r):
    _, q, k, qw, kw, c, s = rope_inputs(d=d, r=r)
    q, k = q.to(device), k.to(device)
    wb = torch.empty(2, d * 2, device=device)
    wb[0, ::2], wb[1, ::2] = qw.float().to(device), kw.float().to(device)
    qwf, kwf = wb[0, ::2], wb[1, ::2]
    cb, sb = torch.empty(13, r * 2, device=device), torch.empty(13, r * 2, device=device)
    cb[:, ::2], sb[:, ::2] = c.to(device), s.to(device)
    out, _ = vw.paper_qk_rmsnorm_rope(q, k, qwf, kwf, cos=cb[:, ::2], sin=sb[:, ::2], enabled=True)
    torch.testing.assert_close(out.cpu(), ow.qk_rope(q.cpu(), qw.float(), 1e-6, c, s), atol=.032, rtol=.02)
    qo, ko = vw.paper_qk_rmsnorm_rope(q[:0], k[:0], qwf, kwf, enabled=True)
    assert qo.shape == ko.shape == (0, 7, d)


@torch.no_grad()
def test_rope_3d_tables_c4_geometry(device):
    """3D RoPE (t,h,w) over 44/42/42 dims, theta 1e4, on a 2x45x80 slab of the C4 grid."""
    cos, sin = vw.rope_tables_3d(2, 45, 80, device=device)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(7200, 4, 128, generator=g).bfloat16()
    w = torch.ones(128, dtype=torch.bfloat16)
    out, _ = vw.paper_qk_rmsnorm_rope(q.to(device), q.to(device), w.to(device), w.to(device),
                                      1e-6, cos, sin, enabled=True)
    expected = ow.qk_rope(q, w, 1e-6, cos.cpu(), sin.cpu())
    torch.testing.assert_close(out.cpu(), expected, atol=.032, rtol=.02)
    assert ((out.cpu().float() - expected.float()).norm() / expected.float().norm()) < 2e-3


@torch.no_grad()
@pytest.mark.parametrize("rows,chunk0,gated", [(1200, 0, True), (1000, 3, False)])
def test_mxfp8_output_equals_quantized_bf16_output(device, rows, chunk0, gated):
    """The quantizing epilogue writes exactly the bytes quantize_activation writes for the bf16
    output, into chunks chunk0 .. chunk0+H-1 of a wider operand; padding rows stay zero."""
    from vdn_amd import mxfp8 as vm
    torch.manual_seed(5)
    frames = 4
    layout = vw.SequenceLayout(rows, 0, frames, rows // frames)
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(frames, 1), device=device)
    h = 5
    q, k, v = [torch.randn(rows, h, 128, device=device, dtype=torch.bfloat16) for _ in range(3)]
    gate = torch.rand(rows, h, 1, device=device, dtype=torch.bfloat16) if gated else None
    ref = vw.paper_window_attention(q, k, v, plan, enabled=True, gate=gate)
    width = (chunk0 + h + 1) * 128
    wide = torch.zeros(rows, width, device=device, dtype=torch.bfloat16)
    wide[:, chunk0 * 128:(chunk0 + h) * 128] = ref.reshape(rows, -1)
    rq, rs = vm.launch_quantize(wide)
    codes, scales = vm.empty_activation(rows, width, device)
    # chunks outside the attention's range hold what the reference buffer holds there (zero)
    codes.zero_()
    scales.copy_(rs)
    assert vw.paper_window_attention(q, k, v, plan, enabled=True, gate=gate,
                                     out_mxfp8=(codes, scales, chunk0)) is None
    assert torch.equal(codes, rq)
    assert torch.equal(scales, rs)


@torch.no_grad()
def test_mxfp8_output_rejects_bad_destinations(device):
    from vdn_amd import mxfp8 as vm
    layout = vw.SequenceLayout(256, 0, 2, 128)
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(2, 1), device=device)
    q = torch.randn(256, 4, 128, device=device, dtype=torch.bfloat16)
    codes, scales = vm.empty_activation(256, 4 * 128, device)
    with pytest.raises(ValueError, match="chunk0"):
        vw.paper_window_attention(q, q, q, plan, enabled=True, out_mxfp8=(codes, scales, 1))
    with pytest.raises(ValueError, match="padded"):
        vw.paper_window_attention(q, q, q, plan, enabled=True,
                                  out_mxfp8=(codes[:, :384].contiguous(), scales, 0))
    with pytest.raises(ValueError, match="excludes"):
        vw.paper_window_attention(q, q, q, plan, enabled=True, return_lse=True,
                                  out_mxfp8=(codes, scales, 0))


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("before,after,frames,chunk,radius,anchor",
                         [(3, 4, 7, 3, 1, "both"), (0, 0, 7, 0, 99, "none"),
                          (3, 0, 2, 5, 1, "rows"), (0, 4, 1, 0, 0, "columns")])
@torch.no_grad()
def test_other_head_dims_dense_fp32_oracle(device, d, before, after, frames, chunk, radius,
                                           anchor):
    """head_dim 64 and 256 (paper_window.py:204 accepts 64, 128, 256) against the dense fp32
    oracle at the reference test's tolerances; strided Q/K/V views, global rows, anchors."""
    torch.manual_seed(820 + d)
    layout = vw.SequenceLayout(before + frames * 3 + after, before, frames, 3)
    bounds = vw.window_bounds(frames, radius, chunk)
    backing = torch.randn(layout.seq_len + 5, 3, 9, d, device=device, dtype=torch.bfloat16)
    q, k, v = [backing[:, i, 2:7] for i in range(3)]
    plan = vw.prepare_paper_window_plan(layout, bounds, anchor, device=device)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    s = layout.seq_len
    mask = ow.dense_mask(s, before, frames, 3, bounds, anchor)
    expected, el = ow.attention_dense(q[:s].cpu(), k[:s].cpu(), v[:s].cpu(), mask, d ** -.5)
    got = out[:s].float().cpu()
    assert out.shape == q.shape
    torch.testing.assert_close(got, expected, atol=.009, rtol=.015)
    assert ((got - expected).norm() / expected.norm()) < .004
    torch.testing.assert_close(lse[:s].cpu(), el, atol=3e-5, rtol=3e-6)
    assert out[s:].count_nonzero() == 0


@pytest.mark.parametrize("d", [64, 256])
@torch.no_grad()
def test_other_head_dims_partial_blocks_tails_and_gate(device, d):
    """300-token frames: 44-row last query blocks, key intervals ending inside a tile (tiles
    of 128 keys for d = 64, 64 for d = 256); the fused gate against the separate product."""
    torch.manual_seed(32 + d)
    frames, spatial = 3, 300
    layout = vw.SequenceLayout(frames * spatial, 0, frames, spatial)
    bounds = vw.window_bounds(frames, 1)
    q, k, v = [torch.randn(layout.seq_len, 2, d, device=device, dtype=torch.bfloat16)
               for _ in range(3)]
    plan = vw.prepare_paper_window_plan(layout, bounds, device=device)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    mask = ow.dense_mask(layout.seq_len, 0, frames, spatial, bounds, "none")
    expected, el = ow.attention_dense(q.cpu(), k.cpu(), v.cpu(), mask, d ** -.5)
    torch.testing.assert_close(out.float().cpu(), expected, atol=.009, rtol=.015)
    torch.testing.assert_close(lse.cpu(), el, atol=3e-5, rtol=3e-6)
    gate = torch.rand(layout.seq_len, 2, device=device).to(torch.bfloat16)
    gated = vw.paper_window_attention(q, k, v, plan, enabled=True, gate=gate)
    assert torch.equal(gated, (out.float() * gate[..., None].float()).to(torch.bfloat16))


@torch.no_grad()
def test_other_head_dims_reject_mxfp8_output(device):
    from vdn_amd import mxfp8 as vm
    layout = vw.SequenceLayout(6, 0, 2, 3)
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(2, 1), device=device)
    q = torch.randn(6, 2, 64, device=device, dtype=torch.bfloat16)
    codes, scales = vm.empty_activation(6, 256, device)
    with pytest.raises(ValueError, match="head_dim 128"):
        vw.paper_window_attention(q, q, q, plan, enabled=True, out_mxfp8=(codes, scales, 0))
    with pytest.raises(ValueError):
        bad = torch.randn(6, 2, 96, device=device, dtype=torch.bfloat16)
        vw.paper_window_attention(bad, bad, bad, plan, enabled=True)


@pytest.mark.parametrize("before,after,frames,chunk,radius,anchor",
                         [(3, 4, 7, 3, 1, "both"), (0, 0, 7, 0, 99, "none"),
                          (0, 0, 3, 0, 1, "none")])
@pytest.mark.parametrize("d", [64, 128, 256])
@torch.no_grad()
def test_fp16_dense_fp32_oracle(device, d, before, after, frames, chunk, radius, anchor):
    """FP16 activations (paper_window.py:206 accepts BF16 and FP16): fp16 output against the
    dense fp32 oracle of the fp16 inputs at the bf16 tests' tolerances (fp16 holds 3 more
    mantissa bits, so the relative error bound is 4x tighter), LSE as for bf16; the fused
    gate equals the separate fp16 product; padding rows zero."""
    torch.manual_seed(900 + d + frames)
    spatial = 300 if frames == 3 else 3
    layout = vw.SequenceLayout(before + frames * spatial + after, before, frames, spatial)
    bounds = vw.window_bounds(frames, radius, chunk)
    backing = torch.randn(layout.seq_len + 5, 3, 5, d, device=device, dtype=torch.float16)
    q, k, v = [backing[:, i, 1:4] for i in range(3)]
    plan = vw.prepare_paper_window_plan(layout, bounds, anchor, device=device)
    out, lse = vw.paper_window_attention(q, k, v, plan, enabled=True, return_lse=True)
    assert out.dtype == torch.float16 and out.shape == q.shape
    s = layout.seq_len
    mask = ow.dense_mask(s, before, frames, spatial, bounds, anchor)
    expected, el = ow.attention_dense(q[:s].cpu(), k[:s].cpu(), v[:s].cpu(), mask, d ** -.5)
    got = out[:s].float().cpu()
    torch.testing.assert_close(got, expected, atol=.003, rtol=.004)
    assert ((got - expected).norm() / expected.norm()) < 1e-3
    torch.testing.assert_close(lse[:s].cpu(), el, atol=3e-5, rtol=3e-6)
    assert out[s:].count_nonzero() == 0
    gate = torch.rand(q.shape[0], 3, device=device).to(torch.float16)
    gated = vw.paper_window_attention(q, k, v, plan, enabled=True, gate=gate)
    assert torch.equal(gated[:s], out[:s] * gate[:s, :, None])


@torch.no_grad()
def test_fp16_rejects_mxfp8_output(device):
    from vdn_amd import mxfp8 as vm
    layout = vw.SequenceLayout(6, 0, 2, 3)
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(2, 1), device=device)
    q = torch.randn(6, 2, 128, device=device, dtype=torch.float16)
    codes, scales = vm.empty_activation(6, 256, device)
    with pytest.raises(ValueError, match="bf16"):
        vw.paper_window_attention(q, q, q, plan, enabled=True, out_mxfp8=(codes, scales, 0))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("d,r,tables", [(128, 128, torch.float32), (128, 96, torch.bfloat16),
                                        (64, 32, torch.float16), (256, 192, torch.float32),
                                        (128, None, None)])
@torch.no_grad()
def test_rope_fp16_fp32_activations(device, dtype, d, r, tables):
    """FP16 and FP32 activations (paper_qk_rope.py:168-186): the kernel against the oracle's
    rounding points in the activation dtype (fp32: none), with weights of the activation
    dtype (q) and fp32 (k), tables of any dtype cast to the activation dtype; and against the
    eager disabled path on the same device."""
    g = torch.Generator().manual_seed(d + (r or 0))
    t, heads = 29, 5
    storage = (torch.randn(t, 3 * heads * d, generator=g) * 2).to(dtype)
    q = storage[:, :heads * d].view(t, heads, d)
    k = storage[:, heads * d:2 * heads * d].view(t, heads, d)
    qw = (torch.rand(d, generator=g) + 0.5).to(dtype)
    kw = (torch.rand(d, generator=g) + 0.5).float()
    c = s = None
    if r is not None:
        angles = torch.randn(t, r // 2, generator=g) * 3
        c = torch.cat((angles.cos(), angles.cos()), 1).to(tables)
        s = torch.cat((angles.sin(), angles.sin()), 1).to(tables)
    dev = lambda x: None if x is None else x.to(device)
    qo, ko = vw.paper_qk_rmsnorm_rope(dev(q), dev(k), dev(qw), dev(kw), 1e-6, dev(c), dev(s),
                                      enabled=True)
    eq, ek = vw.paper_qk_rmsnorm_rope(dev(q), dev(k), dev(qw), dev(kw), 1e-6, dev(c), dev(s),
                                      enabled=False)
    tol = dict(atol=4e-3, rtol=2e-3) if dtype == torch.float16 else dict(atol=2e-5, rtol=2e-5)
    for out, eager, raw, w in ((qo, eq, q, qw), (ko, ek, k, kw)):
        assert out.dtype == dtype and out.is_contiguous() and out.shape == (t, heads, d)
        expected = ow.qk_rope(raw, w, 1e-6, None if c is None else c.float(),
                              None if s is None else s.float())
        torch.testing.assert_close(out.cpu(), expected, **tol)
        torch.testing.assert_close(out, eager, **tol)
