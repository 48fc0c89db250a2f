"""CPU pins of the VDA oracle: closed forms, identities, brute-force loops and the
reference's known answers (no GPU)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import vda as ov
from vdn_amd import vda as vv


def rand_spd_stats(frames, heads, d, s=9, seed=0):
    g = torch.Generator().manual_seed(seed)
    k = F.normalize(torch.randn(frames, heads, s, d, generator=g, dtype=torch.float64), dim=-1)
    A = k.transpose(-1, -2) @ k
    B = torch.randn(frames, heads, d, d, generator=g, dtype=torch.float64) * 0.1
    alpha = (torch.rand(frames, heads, d, generator=g, dtype=torch.float64) * 0.1 + 0.9)
    return A, B, alpha


def test_boundary_plan_reference_kat():
    # tests/test_paper_stack_vda_ops.py:300-307: 35 frames rebased from a 37-frame c1 window
    frames, offset = 35, 1
    bounds = [(lo - offset, hi - offset) for lo, hi in
              ov.window_bounds(frames + 2 * offset, 1, 5)[offset:frames + offset]]
    assert ov.boundary_plan(bounds, frames, 8)["cuts"] == (0, 4, 9, 14, 19, 24, 29, 34, 35)
    plan = vv.paper_boundary_plan(bounds, frames, "cpu", 8)
    assert plan.cuts == (0, 4, 9, 14, 19, 24, 29, 34, 35)


@pytest.mark.parametrize("frames,chunk", [(1, 1), (2, 8), (11, 4), (17, 8), (31, 1), (30, 8)])
def test_product_plan_matches_oracle(frames, chunk):
    bounds = [(f // chunk * chunk - chunk, (f // chunk + 2) * chunk - 1) for f in range(frames)]
    ref = ov.boundary_plan(bounds, frames, chunk)
    plan = vv.paper_boundary_plan(bounds, frames, "cpu", chunk)
    assert plan.cuts == ref["cuts"]
    assert plan.before.tolist() == ref["before"] and plan.after.tolist() == ref["after"]
    assert plan.has_before.tolist() == [int(x) for x in ref["has_before"]]
    assert plan.has_after.tolist() == [int(x) for x in ref["has_after"]]


def test_factor_identities_and_solve_form():
    A, B, alpha = rand_spd_stats(3, 2, 128)
    T, J = ov.factors(A, B, alpha)
    eye = torch.eye(128, dtype=torch.float64)
    M = A + eye
    torch.testing.assert_close((T / alpha[..., None]) @ M, eye.expand_as(M), atol=1e-10, rtol=0)
    torch.testing.assert_close(J @ M, B, atol=1e-10, rtol=0)
    S = torch.randn(2, 128, 128, dtype=torch.float64)
    solve = torch.linalg.solve(M[0], (S * alpha[0][:, None, :] + B[0]).transpose(-1, -2)).transpose(-1, -2)
    torch.testing.assert_close(S @ T[0] + J[0], solve, atol=1e-10, rtol=1e-10)


@pytest.mark.parametrize("radius", [0, 1, 2])
def test_scan_gather_closed_form_identity_transitions(radius):
    frames, h, d = 9, 2, 128
    B = torch.randn(frames, h, d, d, dtype=torch.float64)
    T, J = ov.factors(torch.zeros(frames, h, d, d, dtype=torch.float64), B)
    prefix, suffix = ov.scan(T, J)
    bounds = ov.window_bounds(frames, radius)
    state = ov.gather(prefix, suffix, torch.ones(frames, h, d, dtype=torch.float64), bounds)
    for f, (lo, hi) in enumerate(bounds):
        expect = sum((B[u] for u in range(frames) if u < lo or u > hi), torch.zeros_like(B[0]))
        torch.testing.assert_close(state[f], expect, atol=1e-10, rtol=0)


@pytest.mark.parametrize("frames,chunk", [(11, 4), (17, 8), (6, 1)])
def test_compact_bank_equals_full_banks_at_cuts(frames, chunk):
    A, B, alpha = rand_spd_stats(frames, 1, 128, seed=frames)
    T, J = ov.factors(A, B, alpha)
    seed = torch.randn(1, 128, 128, dtype=torch.float64) * 0.3
    prefix, suffix = ov.scan(T, J, seed)
    bounds = [(f // chunk * chunk - chunk, (f // chunk + 2) * chunk - 1) for f in range(frames)]
    plan = ov.boundary_plan(bounds, frames, chunk)
    bank = ov.compact_bank(prefix, suffix, plan["cuts"])
    # composing each chunk's factors reproduces the bank (the paper's compose + scan)
    cuts = plan["cuts"]
    state = seed.clone()
    for c in range(len(cuts) - 1):
        for f in range(cuts[c], cuts[c + 1]):
            state = state @ T[f] + J[f]
        torch.testing.assert_close(bank[0, c], state, atol=1e-9, rtol=1e-9)


def test_gather_product_and_log_prefix_forms_agree():
    frames, h, d = 7, 2, 128
    A, B, alpha = rand_spd_stats(frames, h, d, seed=3)
    T, J = ov.factors(A, B, alpha)
    prefix, suffix = ov.scan(T, J)
    bounds = ov.window_bounds(frames, 1)
    prod_form = ov.gather(prefix, suffix, alpha, bounds)
    lp = torch.cat([torch.zeros_like(alpha[:1]), alpha.log().cumsum(0)])
    for f, (lo, hi) in enumerate(bounds):
        st = torch.zeros_like(prefix[0])
        if lo > 0:
            st = st + prefix[lo - 1] * torch.exp(lp[f + 1] - lp[lo])[..., None, :]
        if hi + 1 < frames:
            st = st + suffix[hi + 1] * torch.exp(lp[hi + 1] - lp[f])[..., None, :]
        torch.testing.assert_close(prod_form[f], st, atol=1e-12, rtol=1e-10)


def test_statistics_symmetry_and_definition():
    g = torch.Generator().manual_seed(2)
    k = ov.bf16(F.normalize(torch.randn(2, 3, 33, 128, generator=g), dim=-1))
    v = ov.bf16(torch.randn(2, 3, 33, 128, generator=g))
    beta = ov.bf16(torch.rand(2, 3, 33, generator=g))
    A, B = ov.statistics(k, v, beta)
    torch.testing.assert_close(A, A.transpose(-1, -2), atol=0, rtol=0)
    direct = torch.einsum("fhs,fhsi,fhsj->fhij", beta.double(), k.double(), k.double())
    torch.testing.assert_close(A, direct, atol=1e-12, rtol=1e-12)
    vb = (v.double() * beta.double()[..., None]).to(torch.bfloat16).double()
    direct_b = torch.einsum("fhsi,fhsj->fhij", vb, k.double()).to(torch.bfloat16).double()
    torch.testing.assert_close(B, direct_b, atol=0, rtol=0)
    assert torch.linalg.eigvalsh(A + torch.eye(128, dtype=torch.float64)).min() > 0.999


def c1_inputs(alpha_case, seed=0):
    """F=4 frames x 16x16 tokens, 8 heads, head_dim 64, fp32."""
    frames, spatial, h, d = 4, 256, 8, 64
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(frames * spatial, h, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(frames * spatial, h, d, generator=g), dim=-1)
    v = torch.randn(frames * spatial, h, d, generator=g)
    beta = torch.sigmoid(torch.randn(frames * spatial, h, generator=g))
    if alpha_case == "ones":
        alpha = torch.ones(frames, h, d)
    else:  # FrameKDAAlpha with a zero data path: exp(-A * dt), A ~ U(1,16), dt log-uniform
        a = torch.empty(h).uniform_(1, 16, generator=g)
        dt = torch.exp(torch.rand(h * d, generator=g) * (torch.log(torch.tensor(0.1))
                       - torch.log(torch.tensor(0.001))) + torch.log(torch.tensor(0.001)))
        alpha = torch.exp(-a[:, None] * dt.view(h, d)).expand(frames, h, d).contiguous()
    gate = torch.ones(frames * spatial, h, d)
    return q, k, v, beta, gate, alpha, frames, spatial


@pytest.mark.parametrize("alpha_case", ["ones", "kda"])
def test_c1_eager_fp32_matches_independent_fp64(alpha_case):
    q, k, v, beta, gate, alpha, frames, spatial = c1_inputs(alpha_case)
    bounds = ov.window_bounds(frames, 1)
    w = torch.ones(64)
    out32 = ov.eager_branch_fp32(q, k, v, beta, gate, alpha, bounds, frames, spatial, w)
    out64 = ov.eager_branch_fp64(q, k, v, beta, gate, alpha, bounds, frames, spatial, w)
    rel = (out32.double() - out64).norm() / out64.norm()
    assert rel < 4e-3, rel.item()
    assert rel < 1e-4, rel.item()  # fp32 vs fp64 of the same algorithm


def test_paper_branch_oracle_matches_eager_in_float64():
    """The bf16-path oracle (rounding points of the paper kernels) against the eager body
    fed the same bf16 inputs: the reference's branch-vs-fp64 bound."""
    frames, spatial, h, d = 5, 7, 2, 128
    g = torch.Generator().manual_seed(11)
    raw = [ov.bf16(torch.randn(frames * spatial, h, d, generator=g)) for _ in range(3)]
    beta = ov.bf16(torch.rand(frames * spatial, h, generator=g))
    gate = ov.bf16(torch.rand(frames * spatial, h, d, generator=g))
    alpha = torch.rand(frames, h, d, generator=g) * 0.2 + 0.8
    w = torch.rand(d, generator=g) + 0.5
    bounds = ov.window_bounds(frames, 1)
    out, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6)
    ref = ov.eager_branch_fp64(*raw, beta, gate, alpha, bounds, frames, spatial, w)
    rel = (out - ref).norm() / ref.norm()
    assert rel < 4e-3, rel.item()


# ------------------------------------------------------------------- short conv ----

def _conv_operands(frames, fh, fw, h, seed, d=128):
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randn(frames * fh * fw, h, d, generator=g)
    w_sp = torch.randn(h * d, 5, 5, generator=g) / 5
    w_tm = torch.randn(h * d, 5, generator=g) / 5 ** 0.5
    return tokens, w_sp, w_tm


@pytest.mark.parametrize("frames,fh,fw", [(1, 1, 1), (3, 4, 6), (6, 5, 3)])
@pytest.mark.parametrize("l2", [False, True])
def test_short_conv_matches_torch_convolutions(frames, fh, fw, l2):
    """The shifted-sum restatement against torch's depthwise conv2d / conv1d in float64
    (cross-correlation, zero padding 2, groups = channels), then SiLU / L2 in float64."""
    h, d = 2, 16
    tokens, w_sp, w_tm = _conv_operands(frames, fh, fw, h, frames + fh, d)
    c = h * d
    got = ov.short_conv_prepare(tokens, frames, fh, fw, w_sp, w_tm, l2, round_spatial=False)
    vol = tokens.double().reshape(frames, fh, fw, c).permute(0, 3, 1, 2)
    sp = F.conv2d(vol, w_sp.double()[:, None], padding=2, groups=c)        # [F, C, fh, fw]
    seq = sp.permute(2, 3, 1, 0).reshape(fh * fw, c, frames)                # [S, C, F]
    tm = F.conv1d(seq, w_tm.double()[:, None], padding=2, groups=c)         # [S, C, F]
    y = F.silu(tm.permute(2, 0, 1).reshape(frames, fh * fw, h, d))
    if l2:
        y = y / y.square().sum(-1, keepdim=True).clamp_min(1e-12).sqrt()
    torch.testing.assert_close(got, y.permute(0, 2, 1, 3), atol=1e-12, rtol=1e-12)


def test_short_conv_rounds_the_spatial_output_to_bf16():
    """round_spatial rounds the spatial conv's output before the temporal taps: equal to
    the unrounded path fed bf16-rounded spatial values (a temporal identity makes the
    difference visible as exactly the bf16 rounding of the spatial sum)."""
    frames, fh, fw, h, d = 3, 4, 5, 1, 8
    tokens, w_sp, _ = _conv_operands(frames, fh, fw, h, 3, d)
    w_tm = torch.zeros(h * d, 5)
    w_tm[:, 2] = 1
    rounded = ov.short_conv_prepare(tokens, frames, fh, fw, w_sp, w_tm, False)
    exact = ov.short_conv_prepare(tokens, frames, fh, fw, w_sp, w_tm, False, round_spatial=False)
    vol = tokens.double().reshape(frames, fh, fw, h * d).permute(0, 3, 1, 2)
    sp = F.conv2d(vol, w_sp.double()[:, None], padding=2, groups=h * d)
    sp16 = sp.float().bfloat16().double().permute(0, 2, 3, 1).reshape(frames, fh * fw, h, d)
    torch.testing.assert_close(rounded, F.silu(sp16).permute(0, 2, 1, 3), atol=1e-12, rtol=1e-12)
    assert not torch.equal(rounded, exact)


def test_short_conv_unit_impulse_is_prepare():
    """Unit-impulse spatial and temporal weights reduce the short conv to paper_prepare's
    SiLU / L2 (bf16 inputs survive the spatial rounding exactly)."""
    frames, fh, fw, h, d = 4, 3, 5, 2, 128
    tokens = _conv_operands(frames, fh, fw, h, 5)[0].bfloat16().double()
    w_sp = torch.zeros(h * d, 5, 5)
    w_sp[:, 2, 2] = 1
    w_tm = torch.zeros(h * d, 5)
    w_tm[:, 2] = 1
    for l2 in (False, True):
        got = ov.short_conv_prepare(tokens, frames, fh, fw, w_sp, w_tm, l2)
        torch.testing.assert_close(got, ov.prepare(tokens, frames, fh * fw, l2), atol=0, rtol=0)


def test_short_conv_temporal_loop_of_the_reference_test():
    """The reference test's own temporal oracle (test_paper_stack_vda_ops.py:43-49):
    acc[t] += x[t + j - 2] * w[:, j] for in-range frames, on a spatial identity."""
    frames, fh, fw, h, d = 7, 2, 3, 1, 16
    tokens, _, w_tm = _conv_operands(frames, fh, fw, h, 11, d)
    w_sp = torch.zeros(h * d, 5, 5)
    w_sp[:, 2, 2] = 1
    x = tokens.bfloat16().double().reshape(frames, fh * fw, h * d)
    acc = torch.zeros_like(x)
    for t in range(frames):
        for j in range(5):
            if 0 <= t + j - 2 < frames:
                acc[t] += x[t + j - 2] * w_tm[:, j].double()
    expected = F.silu(acc).reshape(frames, fh * fw, h, d).permute(0, 2, 1, 3)
    got = ov.short_conv_prepare(tokens.bfloat16().double(), frames, fh, fw, w_sp, w_tm, False)
    torch.testing.assert_close(got, expected, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("d", [16, 64])
def test_paper_branch_oracle_small_head_dim_matches_eager(d):
    """The bf16-path oracle at head dims below 128 (the reference's eager body takes any d,
    delta_rule.py:45-60) against the float64 eager body on the same bf16 inputs."""
    frames, spatial, h = 4, 9, 2
    g = torch.Generator().manual_seed(d)
    raw = [ov.bf16(torch.randn(frames * spatial, h, d, generator=g)) for _ in range(3)]
    beta = ov.bf16(torch.rand(frames * spatial, h, generator=g))
    gate = ov.bf16(torch.rand(frames * spatial, h, d, generator=g))
    alpha = torch.rand(frames, h, d, generator=g) * 0.2 + 0.8
    w = torch.rand(d, generator=g) + 0.5
    bounds = ov.window_bounds(frames, 1)
    out, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6)
    ref = ov.eager_branch_fp64(*raw, beta, gate, alpha, bounds, frames, spatial, w)
    assert out.shape == (frames * spatial, h * d)
    rel = (out - ref).norm() / ref.norm()
    assert rel < 4e-3, rel.item()
