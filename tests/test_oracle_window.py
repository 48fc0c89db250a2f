"""CPU pins of the window-attention / RoPE oracle and of the plan's interval form."""
import pytest
import torch
import torch.nn.functional as F

from oracle import window as ow
from vdn_amd import window as vw

LAYOUTS = [(0, 0), (3, 0), (0, 4), (3, 4)]
GEOMETRY = [(1, 0, 0), (2, 5, 1), (7, 3, 0), (7, 3, 1), (7, 0, 1), (7, 5, 1), (7, 0, 99)]


def layout_of(before, after, frames, tpf=3):
    return vw.SequenceLayout(before + frames * tpf + after, before, frames, tpf,
                             text_start=0 if before else frames * tpf, text_len=before or after)


@pytest.mark.parametrize("before,after", LAYOUTS)
@pytest.mark.parametrize("frames,chunk,radius", GEOMETRY)
@pytest.mark.parametrize("anchor", ["none", "rows", "columns", "both"])
def test_plan_matches_dense_mask(before, after, frames, chunk, radius, anchor):
    layout = layout_of(before, after, frames)
    bounds = vw.window_bounds(frames, radius, chunk)
    plan = vw.prepare_paper_window_plan(layout, bounds, anchor, max_gather_rows=2 * layout.seq_len,
                                        max_query_rows=5)
    expected = ow.dense_mask(layout.seq_len, layout.video_start, frames, 3, bounds, anchor)
    # reference pass structure (tests/test_paper_stack_attention_window.py:37-66)
    seen = []
    for p in plan.passes:
        assert p.query_rows.numel() <= 5
        for g in p.groups:
            for a, b in g.query_ranges:
                seen.extend(range(a, b))
    assert sorted(seen) == list(range(layout.seq_len))
    # the kernel's interval form covers exactly the mask, block by block
    dp = plan.device_plan
    actual = torch.zeros_like(expected)
    covered = []
    for q0, q_end, gi in dp.blocks[:dp.nblocks].tolist():
        rows = range(q0, min(q0 + vw.BLOCK_M, q_end))
        covered.extend(rows)
        for a, b in dp.intervals[gi][:dp.counts[gi]].tolist():
            assert a < b
            for q in rows:
                actual[q, a:b] = True
    assert sorted(covered) == list(range(layout.seq_len))
    assert torch.equal(actual, expected)


def test_clamped_visible_sets_grouped_and_budget_errors():
    plan = vw.prepare_paper_window_plan(vw.SequenceLayout(8, 0, 4, 2), [(-3, 1), (-2, 1), (2, 9), (2, 8)])
    assert len(plan.passes) == 1 and len(plan.passes[0].groups) == 2
    layout = vw.SequenceLayout(21, 0, 7, 3)
    with pytest.raises(ValueError, match="requires 9 gather rows"):
        vw.prepare_paper_window_plan(layout, vw.window_bounds(7, 1), max_gather_rows=8)
    with pytest.raises(ValueError, match="no visible keys"):
        vw.prepare_paper_window_plan(vw.SequenceLayout(3, 0, 1, 3), [(4, 5)])
    plan = vw.prepare_paper_window_plan(vw.SequenceLayout(9, 4, 0, 3), [], max_gather_rows=1,
                                        max_query_rows=2)
    assert len(plan.passes) == 5 and plan.peak_gather_rows == 0
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(7, 99), max_gather_rows=1)
    assert all(p.dense for p in plan.passes)


@pytest.mark.parametrize("kwargs", [{"anchor_frames": "bad"}, {"max_gather_rows": 0},
                                    {"max_query_rows": -1}])
def test_invalid_plan_options(kwargs):
    with pytest.raises(ValueError):
        vw.prepare_paper_window_plan(vw.SequenceLayout(6, 0, 2, 3), [(0, 1)] * 2, **kwargs)


@pytest.mark.parametrize("bounds", [[], [(0, 1)], [(2, 1), (0, 1)], [(0., 1), (0, 1)]])
def test_invalid_bounds(bounds):
    with pytest.raises(ValueError):
        vw.prepare_paper_window_plan(vw.SequenceLayout(6, 0, 2, 3), bounds)


def test_disabled_and_grad_contracts():
    with pytest.raises(RuntimeError, match="disabled"):
        vw.paper_window_attention(None, None, None, None)
    with torch.enable_grad(), pytest.raises(RuntimeError, match="inference-only"):
        vw.paper_window_attention(None, None, None, None, enabled=True)


def test_dense_oracle_closed_form_constant_values():
    layout = vw.SequenceLayout(45, 2, 13, 3)
    bounds = vw.window_bounds(13, 1, 3)
    mask = ow.dense_mask(45, 2, 13, 3, bounds, "columns")
    q = torch.zeros(45, 2, 128)
    v = torch.arange(45, dtype=torch.float32)[:, None, None].expand(45, 2, 128)
    out, lse = ow.attention_dense(q, q, v, mask, 128 ** -.5)
    expected = (mask.float() @ torch.arange(45).float()) / mask.sum(-1)
    torch.testing.assert_close(out[:, 0, 0], expected, rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(lse[:, 0], mask.sum(-1).float().log(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("anchor", ["none", "both"])
def test_dense_oracle_matches_per_frame_reference(anchor):
    torch.manual_seed(5)
    layout = vw.SequenceLayout(3 + 7 * 4 + 2, 3, 7, 4)
    bounds = vw.window_bounds(7, 1, 3)
    q, k, v = (torch.randn(layout.seq_len, 2, 128) for _ in range(3))
    ref = ow.window_softmax_reference(q, k, v, layout, bounds, 128 ** -.5, anchor)
    mask = ow.dense_mask(layout.seq_len, 3, 7, 4, bounds, anchor)
    out, _ = ow.attention_dense(q, k, v, mask, 128 ** -.5)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


def rope_inputs(r=96, t=13, seed=194):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, 7, 128, generator=g).to(torch.bfloat16)
    w = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    angles = torch.randn(t, r // 2, generator=g)
    cos = torch.cat((angles.cos(), angles.cos()), 1)
    sin = torch.cat((angles.sin(), angles.sin()), 1)
    return x, w, cos, sin


def test_rope_oracle_rounding_traps_and_complex_rotation():
    g = torch.Generator().manual_seed(715)
    x = torch.ones(3, 7, 128, dtype=torch.bfloat16)
    w = (torch.rand(128, generator=g) * 1.7 + .1).bfloat16()
    angles = torch.randn(3, 96, generator=g)
    c, s = angles.cos(), angles.sin()
    exact = ow.qk_rope(x, w, .25, c, s)
    assert torch.count_nonzero(exact != ow.qk_rope(x, w, .25, c, s, round_norm=False)) > 100
    assert torch.count_nonzero(exact != ow.qk_rope(x, w, .25, c, s, round_products=False)) > 100
    # rotate-half with equal-angle halves is complex multiplication (float64 reference)
    x, w, cos, sin = rope_inputs()
    n = ow.qk_rope(x, w, 1e-6)  # norm only
    unrounded = ow.qk_rope(x, w, 1e-6, cos, sin, round_products=False)
    cplx = ow.rope_complex_fp64(n.float(), cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float())
    torch.testing.assert_close(unrounded.double(), cplx.to(torch.bfloat16).double(), rtol=8e-3, atol=1e-2)
    rel = (unrounded.double() - cplx).norm() / cplx.norm()
    assert rel < 4e-3


def test_rope_norm_only_equals_rms_norm():
    x, w, _, _ = rope_inputs()
    ref = F.rms_norm(x.float(), (128,), w.float(), 1e-6).to(torch.bfloat16)
    out = ow.qk_rope(x, w, 1e-6)
    assert (out.float() - ref.float()).abs().max() <= 2 ** -7 * ref.float().abs().max()


def test_rope_tables_3d_match_oracle():
    c1, s1 = vw.rope_tables_3d(3, 4, 5, dtype=torch.float64)
    c2, s2 = ow.rope_tables_3d(3, 4, 5)
    torch.testing.assert_close(c1, c2, rtol=0, atol=1e-12)
    torch.testing.assert_close(s1, s2, rtol=0, atol=1e-12)
    assert c1.shape == (60, 128)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@torch.no_grad()
def test_rope_disabled_eager_path_matches_oracle(dtype):
    """paper_qk_rmsnorm_rope(enabled=False) is the reference's eager path on the tensors' own
    device (paper_qk_rope.py:82-95, 168-176): bit-equal to the oracle on the rounding-trap
    input (its mean square is exact) and within one rounding of the activation dtype on
    random strided inputs, for each activation dtype; fp32 and activation-dtype weights."""
    g = torch.Generator().manual_seed(715)
    x = torch.ones(3, 7, 128, dtype=dtype)
    w = (torch.rand(128, generator=g) * 1.7 + .1).to(dtype)
    angles = torch.randn(3, 96, generator=g)
    c, s = angles.cos(), angles.sin()
    qo, ko = vw.paper_qk_rmsnorm_rope(x, x, w, w.float(), .25, c, s)
    assert qo.dtype == dtype and torch.equal(qo, ow.qk_rope(x, w, .25, c, s))
    assert torch.equal(ko, ow.qk_rope(x, w.float(), .25, c, s))
    storage = torch.randn(13, 3 * 7 * 128, generator=g).to(dtype)
    q, k = storage[:, :896].view(13, 7, 128), storage[:, 896:1792].view(13, 7, 128)
    ang = torch.randn(13, 64, generator=g)
    cos, sin = torch.cat((ang.cos(), ang.cos()), 1), torch.cat((ang.sin(), ang.sin()), 1)
    qo, ko = vw.paper_qk_rmsnorm_rope(q, k, w, w, 1e-6, cos, sin)
    for out, raw in ((qo, q), (ko, k)):
        exp = ow.qk_rope(raw, w, 1e-6, cos, sin).float()
        ulp = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 2 ** -22}[dtype]
        assert ((out.float() - exp).abs() <= 2 * ulp * exp.abs() + 1e-6).all()
    n_only, _ = vw.paper_qk_rmsnorm_rope(q, k, w, w, 1e-6)
    torch.testing.assert_close(n_only, ow.qk_rope(q, w, 1e-6), atol=0, rtol=2 ** -6)
    with torch.enable_grad(), pytest.raises(RuntimeError, match="inference-only"):
        vw.paper_qk_rmsnorm_rope(q, k, w, w, 1e-6, cos, sin)
