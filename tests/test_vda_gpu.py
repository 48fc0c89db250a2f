"""GPU parity of the VDA kernels against the float64 oracle, at the reference test's
tolerances (tests/test_paper_stack_vda_ops.py, test_paper_stack_vda_factor.py)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import vda as ov
from vdn_amd import vda as vv

pytestmark = pytest.mark.gpu


def close_rel(a, b, limit):
    err = (a.double().cpu() - b.double().cpu()).norm() / b.double().cpu().norm().clamp_min(1e-20)
    assert err.item() < limit, err.item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("frames,spatial", [(1, 1), (3, 7), (17, 12)])
@pytest.mark.parametrize("l2", [False, True])
def test_prepare(device, dtype, frames, spatial, l2):
    torch.manual_seed(711)
    raw = torch.randn(frames * spatial, 2, 128, dtype=dtype)
    out = vv.paper_prepare(raw.to(device), frames=frames, spatial=spatial, l2norm=l2)
    ref = ov.prepare(raw, frames, spatial, l2)
    assert out.is_contiguous() and out.shape == (frames, 2, spatial, 128)
    if dtype == torch.bfloat16:
        torch.testing.assert_close(out.cpu(), ref.to(dtype), atol=0., rtol=0.008)
    else:
        close_rel(out, ref, 5e-7)


@pytest.mark.parametrize("beta_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("s", [1, 33, 129, 1008])
def test_statistics(device, beta_dtype, s):
    torch.manual_seed(s)
    k = F.normalize(torch.randn(3, 2, s, 128), dim=-1).to(torch.bfloat16)
    v = torch.randn_like(k)
    beta = torch.rand(3, 2, s).to(beta_dtype)
    a, b = vv.paper_statistics(k.to(device), v.to(device), beta.to(device))
    ra, rb = ov.statistics(k, v, beta)
    assert a.dtype == b.dtype == torch.float32
    close_rel(a, ra, 5e-7)
    close_rel(b, rb, 1e-4)
    torch.testing.assert_close(a, a.transpose(-1, -2), atol=2e-6, rtol=1e-6)


def test_statistics_correlated_keys_spd(device):
    s = 1008
    base = torch.randn(2, 3, 1, 128)
    k = F.normalize(base + torch.randn(2, 3, s, 128) * .01, dim=-1).bfloat16()
    v = torch.randn_like(k) * 10
    beta = torch.rand(2, 3, s, dtype=torch.bfloat16)
    a, b = vv.paper_statistics(k.to(device), v.to(device), beta.to(device))
    ref = (k.double() * beta.double()[..., None]).transpose(-1, -2) @ k.double()
    close_rel(a, ref, 5e-7)
    assert torch.linalg.eigvalsh(a.double().cpu() + torch.eye(128, dtype=torch.float64)).min() > .999
    t, inj = vv.paper_delta_factors(a, b)
    inv = torch.linalg.inv(ref + torch.eye(128, dtype=torch.float64))
    close_rel(t, inv, 3e-5)
    close_rel(inj, b.double().cpu() @ inv, 3e-5)


def test_statistics_from_projections_equals_prepare_then_statistics(device):
    frames, spatial, h = 3, 50, 4
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(frames * spatial, 3 * h * 128, generator=g).to(torch.bfloat16).to(device)
    k = qkv[:, h * 128:2 * h * 128].view(-1, h, 128)
    v = qkv[:, 2 * h * 128:].view(-1, h, 128)
    beta = torch.rand(frames * spatial, h, generator=g).to(torch.bfloat16).to(device)
    a1, b1 = vv.statistics_from_projections(k, v, beta, frames, spatial)
    kp = vv.paper_prepare(k, frames=frames, spatial=spatial, l2norm=True)
    vp = vv.paper_prepare(v, frames=frames, spatial=spatial, l2norm=False)
    bp = beta.view(frames, spatial, h).permute(0, 2, 1).contiguous()
    a2, b2 = vv.paper_statistics(kp, vp, bp)
    assert torch.equal(a1, a2) and torch.equal(b1, b2)


def test_factors_fp64(device):
    A, B, alpha = (t.float() for t in _stats(5, 3, seed=1))
    T, J = vv.paper_delta_factors(A.to(device), B.to(device), alpha.to(device))
    rT, rJ = ov.factors(A, B, alpha)
    close_rel(T, rT, 1e-5)
    close_rel(J, rJ, 3e-5)
    T1, _ = vv.paper_delta_factors(A.to(device), B.to(device))
    close_rel(T1, ov.factors(A, B)[0], 1e-5)
    e = vv.paper_delta_factors(torch.empty(0, 128, 128, device=device),
                               torch.empty(0, 128, 128, device=device))
    assert e[0].shape == (0, 128, 128)


def _stats(frames, heads, seed=0, s=9, decay=1.0):
    g = torch.Generator().manual_seed(seed)
    k = F.normalize(torch.randn(frames, heads, s, 128, generator=g), dim=-1)
    A = (k.transpose(-1, -2) @ k).contiguous()
    B = torch.randn(frames, heads, 128, 128, generator=g) * 0.1
    alpha = (torch.rand(frames, heads, 128, generator=g) * 0.1 + 0.9) * decay
    return A, B, alpha


@pytest.mark.parametrize("frames,chunk", [(1, 1), (2, 8), (11, 4), (17, 8), (31, 1)])
@pytest.mark.parametrize("text", [False, True])
@pytest.mark.parametrize("decay", [1., 0.7, 0.001])
def test_scan_and_gather_fp64(device, frames, chunk, text, decay):
    h = 2
    A, B, alpha = _stats(frames, h, seed=frames * 7 + chunk, decay=decay)
    t, inj = vv.paper_delta_factors(A.to(device), B.to(device), alpha.to(device))
    seed = torch.randn(h, 128, 128) * .3 if text else None
    bounds = [(f // chunk * chunk - chunk, (f // chunk + 2) * chunk - 1) for f in range(frames)]
    plan = vv.paper_boundary_plan(bounds, frames, device, chunk)
    bank = vv.paper_boundary_scan(t, inj, plan, None if seed is None else seed.to(device))
    prefix, suffix = ov.scan(t.cpu(), inj.cpu(), seed)
    torch.testing.assert_close(bank[0].double().cpu(), prefix[torch.tensor(plan.cuts[1:]) - 1],
                               atol=3e-6, rtol=3e-5)
    torch.testing.assert_close(bank[1].double().cpu(), suffix[list(plan.cuts[:-1])],
                               atol=3e-6, rtol=3e-5)
    result = vv.paper_gather(bank, alpha.to(device), plan, None if seed is None else seed.to(device),
                             torch.float32)
    expected = ov.gather(prefix, suffix, alpha, bounds, seed)
    torch.testing.assert_close(result.double().cpu(), expected, atol=4e-6, rtol=5e-5)
    assert bank.shape == (2, plan.chunks, h, 128, 128)


def test_gather_zero_decay_irregular_bounds_no_bridge(device):
    frames, h = 9, 1
    t = (torch.eye(128).expand(frames, h, 128, 128).contiguous() * .9)
    inj = torch.randn_like(t)
    alpha = torch.zeros(frames, h, 128)
    bounds = [(max(0, f - f % 3), min(frames - 1, f + 2)) for f in range(frames)]
    plan = vv.paper_boundary_plan(bounds, frames, device, 4)
    seed = torch.randn_like(t[0])
    bank = vv.paper_boundary_scan(t.to(device), inj.to(device), plan, seed.to(device))
    prefix, suffix = ov.scan(t, inj, seed)
    for bridge in (True, False):
        out = vv.paper_gather(bank, alpha.to(device), plan, seed.to(device), torch.float32, bridge)
        ref = ov.gather(prefix, suffix, alpha, bounds, seed, bridge)
        torch.testing.assert_close(out.double().cpu(), ref, atol=5e-6, rtol=1e-5)


def test_epilogue(device):
    r = torch.randn(3, 2, 7, 128, dtype=torch.bfloat16)
    w = torch.rand(128)
    g = torch.rand(21, 2, 128, dtype=torch.bfloat16)
    out = vv.vdn_linear_epilogue(r.to(device), w.to(device), g.to(device), 1e-6)
    ref = ov.epilogue(r, w, g, 1e-6)
    torch.testing.assert_close(out.cpu(), ref.to(out.dtype), atol=0.0078125, rtol=0.008)


def _branch_inputs(frames, spatial, h, seed, text=False):
    g = torch.Generator().manual_seed(seed)
    raw = [torch.randn(frames * spatial, h, 128, generator=g).bfloat16() for _ in range(3)]
    beta = torch.rand(frames * spatial, h, generator=g).bfloat16()
    gate = torch.rand(frames * spatial, h, 128, generator=g).bfloat16()
    alpha = torch.rand(frames, h, 128, generator=g) * 0.2 + 0.8
    w = torch.rand(128, generator=g) + 0.5
    tx = None
    if text:
        tx = (torch.randn(5, h, 128, generator=g).bfloat16(),
              torch.randn(5, h, 128, generator=g).bfloat16(),
              torch.rand(5, h, generator=g).bfloat16())
    return raw, beta, gate, alpha, w, tx


@pytest.mark.parametrize("text", [False, True])
@pytest.mark.parametrize("frames,spatial,chunk,radius", [(11, 7, 4, 1), (9, 70, 8, 1),
                                                         (5, 130, 8, 2)])
def test_branch_against_fp64_oracle(device, text, frames, spatial, chunk, radius):
    raw, beta, gate, alpha, w, tx = _branch_inputs(frames, spatial, 2, frames + spatial, text)
    bounds = ov.window_bounds(frames, radius)
    dev = lambda x: x.to(device)
    out = vv.vda_forward(*map(dev, raw), dev(beta), dev(gate), dev(alpha), bounds, frames, spatial,
                         dev(w), 1e-6, chunk_size=chunk,
                         text=None if tx is None else tuple(map(dev, tx)))
    ref, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6, text=tx)
    assert out.dtype == torch.bfloat16 and out.shape == (frames * spatial, 2 * 128)
    close_rel(out, ref, 0.004)


def test_branch_on_fused_qkv_strides(device):
    """Raw q/k/v as column slices of one fused projection output (the block's layout)."""
    frames, spatial, h = 4, 40, 3
    g = torch.Generator().manual_seed(8)
    qkv = torch.randn(frames * spatial, 3 * h * 128, generator=g).bfloat16()
    raw = [qkv[:, i * h * 128:(i + 1) * h * 128].view(-1, h, 128) for i in range(3)]
    beta = torch.rand(frames * spatial, h, generator=g).bfloat16()
    gate = torch.rand(frames * spatial, h, 128, generator=g).bfloat16()
    alpha = torch.rand(frames, h, 128, generator=g) * 0.2 + 0.8
    w = torch.ones(128)
    bounds = ov.window_bounds(frames, 1)
    qd = qkv.to(device)
    rd = [qd[:, i * h * 128:(i + 1) * h * 128].view(-1, h, 128) for i in range(3)]
    out = vv.vda_forward(*rd, beta.to(device), gate.to(device), alpha.to(device), bounds, frames,
                         spatial, w.to(device), 1e-6)
    ref, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6)
    close_rel(out, ref, 0.004)


def test_c3_full_shape_sampled_heads(device):
    """C3: 30 frames x 3600 tokens, 40 heads, d 128, window +-1 frame. Heads are independent,
    so parity is checked on 2 of the 40 heads against the float64 oracle."""
    frames, spatial, h = 30, 3600, 40
    g = torch.Generator().manual_seed(3)
    n = frames * spatial
    q = F.normalize(torch.randn(n, h, 128, generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(n, h, 128, generator=g), dim=-1).bfloat16()
    v = torch.randn(n, h, 128, generator=g).bfloat16()
    beta = torch.sigmoid(torch.randn(n, h, generator=g)).bfloat16()
    gate = torch.sigmoid(torch.randn(n, h, 128, generator=g)).bfloat16()
    a = torch.empty(h).uniform_(1, 16, generator=g)
    dt = torch.exp(torch.rand(h, 128, generator=g) * (torch.log(torch.tensor(0.1))
                   - torch.log(torch.tensor(0.001))) + torch.log(torch.tensor(0.001)))
    alpha = torch.exp(-a[:, None] * dt).expand(frames, h, 128).contiguous()
    w = torch.ones(128)
    bounds = ov.window_bounds(frames, 1)
    out = vv.vda_forward(q.to(device), k.to(device), v.to(device), beta.to(device),
                         gate.to(device), alpha.to(device), bounds, frames, spatial, w.to(device),
                         1e-6)
    assert bool(torch.isfinite(out).all())
    heads = [0, 29]
    sel = lambda x: x[:, heads].contiguous()
    ref, _ = ov.paper_branch(sel(q), sel(k), sel(v), sel(beta), sel(gate), alpha[:, heads], bounds,
                             frames, spatial, w, 1e-6)
    got = out.view(n, h, 128)[:, heads].reshape(n, -1)
    close_rel(got, ref, 0.004)


@torch.no_grad()
@pytest.mark.parametrize("chunk0", [0, 2])
def test_readout_mxfp8_equals_quantized_bf16_readout(device, chunk0):
    """The quantizing readout epilogue writes exactly the bytes quantize_activation writes for
    the bf16 readout, into chunks chunk0 .. chunk0+H-1; padding rows read as zero."""
    from vdn_amd import mxfp8 as vm
    frames, spatial, h = 3, 50, 3
    g = torch.Generator().manual_seed(21)
    n = frames * spatial
    q = torch.randn(n, h, 128, generator=g).bfloat16().to(device)
    state = (torch.randn(frames, h, 128, 128, generator=g) * 0.1).bfloat16().to(device)
    gate = torch.rand(n, h, 128, generator=g).bfloat16().to(device)
    w = (torch.rand(128, generator=g) + 0.5).to(device)
    ref = vv.linear_readout(q, state, w, gate, 1e-6, frames, spatial)
    width = (chunk0 + h) * 128
    wide = torch.zeros(n, width, device=device, dtype=torch.bfloat16)
    wide[:, chunk0 * 128:] = ref
    rq, rs = vm.launch_quantize(wide)
    codes, scales = vm.empty_activation(n, width, device)
    codes.zero_()
    scales.copy_(rs)
    assert vv.linear_readout(q, state, w, gate, 1e-6, frames, spatial,
                             out_mxfp8=(codes, scales, chunk0)) is None
    assert torch.equal(codes, rq)
    assert torch.equal(scales, rs)


def _gate_operands(n, h, g, device):
    down = (torch.randn(n, 208, generator=g) * 0.5).bfloat16().to(device)[:, 80:]
    up_w = (torch.randn(h * 128, 128, generator=g) * 0.1).bfloat16().to(device)
    up_b = (torch.randn(h * 128, generator=g) * 0.5).bfloat16().to(device)
    return down, up_w, up_b


@torch.no_grad()
def test_gated_readout_forms_the_output_gate(device):
    """With q = ones, state = identity and unit weights the readout returns the gate itself
    (RMSNorm of a constant row is 1 - 5e-7, which bf16 rounding absorbs), so the gate formed
    in the kernel is compared with OutputGate's torch composition sigmoid(up(down)) on a
    strided down view: equal but for one-ulp bf16 flips where the two GEMMs' fp32 sums
    straddle a rounding boundary."""
    frames, spatial, h = 2, 131, 3
    n = frames * spatial
    g = torch.Generator().manual_seed(5)
    down, up_w, up_b = _gate_operands(n, h, g, device)
    q = torch.ones(n, h, 128, dtype=torch.bfloat16, device=device)
    state = torch.eye(128).expand(frames, h, 128, 128).bfloat16().contiguous().to(device)
    w = torch.ones(128, device=device)
    out = vv.linear_readout(q, state, w, vv.OutputGateProjection(down, up_w, up_b), 1e-6, frames,
                            spatial, activate_q=False)
    ref = torch.sigmoid(F.linear(down, up_w, up_b))
    diff = (out.float() - ref.float()).abs()
    ulp = torch.finfo(torch.bfloat16).eps * ref.float().abs()
    assert bool((diff <= ulp).all()), diff.max().item()
    assert (diff == 0).float().mean().item() > 0.99


@torch.no_grad()
@pytest.mark.parametrize("chunk0", [0, 3])
def test_gated_readout_matches_the_read_gate(device, chunk0):
    """The gated readout against the readout of the torch-formed gate (activated q), in bf16
    and into MXFP8, where it must equal quantize_activation of its own bf16 result."""
    from vdn_amd import mxfp8 as vm
    frames, spatial, h = 3, 70, 3
    n = frames * spatial
    g = torch.Generator().manual_seed(8)
    q = torch.randn(n, h, 128, generator=g).bfloat16().to(device)
    state = (torch.randn(frames, h, 128, 128, generator=g) * 0.1).bfloat16().to(device)
    w = (torch.rand(128, generator=g) + 0.5).to(device)
    down, up_w, up_b = _gate_operands(n, h, g, device)
    gp = vv.OutputGateProjection(down, up_w, up_b)
    gate = torch.sigmoid(F.linear(down, up_w, up_b)).view(n, h, 128)
    ref = vv.linear_readout(q, state, w, gate, 1e-6, frames, spatial)
    got = vv.linear_readout(q, state, w, gp, 1e-6, frames, spatial)
    close_rel(got, ref, 2e-3)
    width = (chunk0 + h) * 128
    wide = torch.zeros(n, width, device=device, dtype=torch.bfloat16)
    wide[:, chunk0 * 128:] = got
    rq, rs = vm.launch_quantize(wide)
    codes, scales = vm.empty_activation(n, width, device)
    codes.zero_()
    scales.copy_(rs)
    assert vv.linear_readout(q, state, w, gp, 1e-6, frames, spatial,
                             out_mxfp8=(codes, scales, chunk0)) is None
    assert torch.equal(codes, rq)
    assert torch.equal(scales, rs)


def test_gated_readout_rejects_bad_operands(device):
    from vdn_amd import _lib
    frames, spatial, h = 1, 16, 2
    n = frames * spatial
    g = torch.Generator().manual_seed(1)
    down, up_w, up_b = _gate_operands(n, h, g, device)
    q = torch.randn(n, h, 128, generator=g).bfloat16().to(device)
    state = torch.zeros(frames, h, 128, 128, dtype=torch.bfloat16, device=device)
    w = torch.ones(128, device=device)
    with pytest.raises(ValueError, match="up_weight"):
        vv.linear_readout(q, state, w, vv.OutputGateProjection(down, up_w[:128], up_b), 1e-6,
                          frames, spatial)
    with pytest.raises(ValueError, match="down"):
        vv.linear_readout(q, state, w, vv.OutputGateProjection(down[:, :64], up_w, up_b), 1e-6,
                          frames, spatial)
    with pytest.raises(RuntimeError, match="exactly one of out and codes"):
        _lib.call("vdn_vda_readout_gated", q.data_ptr(), spatial * q.stride(0), q.stride(1),
                  q.stride(0), 1, state.data_ptr(), w.data_ptr(), 1, 1e-6, down.data_ptr(),
                  down.stride(0), up_w.data_ptr(), up_b.data_ptr(), None, 0, 0, 0, None, None, 0,
                  0, frames, h, spatial, _lib.stream(q.device))


# ------------------------------------------------------------------- short conv ----

def _sep_conv(h, projs, seed):
    torch.manual_seed(seed)
    return vv.LinearAttentionSepConv(h * 128, projs).to(torch.bfloat16)


def _conv_weights(conv, proj):
    w_sp, w_tm = conv.weights(proj, torch.bfloat16)
    return w_sp.float().reshape(-1, 5, 5), w_tm.float()


@pytest.mark.parametrize("frames,fh,fw", [(1, 1, 1), (3, 7, 5), (5, 9, 12), (2, 16, 8),
                                          (6, 10, 17), (4, 6, 9), (9, 8, 8)])
@pytest.mark.parametrize("l2", [False, True])
def test_conv_prepare_against_oracle(device, frames, fh, fw, l2):
    """Fused spatial + temporal short conv, SiLU / L2, frame-major store, against the float64
    restatement with the reference's bf16 rounding of the spatial output, at the reference
    test's bf16 bound (rtol 0.008; test_paper_stack_vda_ops.py:52-54). The reference test
    feeds its oracle the conv2d's own bf16 output; this oracle recomputes it, so where the
    kernel's fp32 spatial sum and the float64 one round to neighbouring bf16 values the
    temporal sum moves by one such step times a tap weight: that is the absolute slack,
    2^-8 * max|spatial| * max|w_tm|, and it may be used by at most 1e-4 of the outputs.
    Frame sizes cover partial 8 x 8 tiles and a frame smaller than the 5 x 5 stencil; the
    frame counts give every remainder of the kernel's frame loop (frames + 2 steps, unrolled
    five times: remainders 3, 4, 0, 2, 3, 1, 1)."""
    h = 2
    conv = _sep_conv(h, ("k",), frames * 31 + fw)
    g = torch.Generator().manual_seed(fh)
    raw = torch.randn(frames * fh * fw, h, 128, generator=g).bfloat16()
    out = vv.paper_prepare(raw.to(device), frames=frames, spatial=fh * fw, l2norm=l2,
                           conv=conv.to(device), proj="k", frame_size=(fh, fw))
    assert out.shape == (frames, h, fh * fw, 128) and out.is_contiguous()
    w_sp, w_tm = _conv_weights(conv.cpu(), "k")
    ref = ov.short_conv_prepare(raw, frames, fh, fw, w_sp, w_tm, l2).to(torch.bfloat16).double()
    vol = raw.double().reshape(frames, fh, fw, h * 128).permute(0, 3, 1, 2)
    spatial = F.conv2d(vol, w_sp.double()[:, None], padding=2, groups=h * 128)
    slack = 2.0 ** -8 * spatial.abs().max().item() * w_tm.abs().max().item()
    diff = (out.cpu().double() - ref).abs()
    outside = diff > 0.008 * ref.abs()
    assert bool((diff <= 0.008 * ref.abs() + slack).all()), diff.max().item()
    assert outside.double().mean().item() <= 1e-4


def test_conv_prepare_on_fused_qkv_strides(device):
    """K and V as strided column slices of one fused projection (the block's layout) give the
    same bytes as the contiguous copies."""
    frames, fh, fw, h = 4, 6, 9, 3
    conv = _sep_conv(h, ("k", "v"), 4).to(device)
    g = torch.Generator().manual_seed(2)
    qkv = torch.randn(frames * fh * fw, 3 * h * 128, generator=g).bfloat16().to(device)
    for i, proj in ((1, "k"), (2, "v")):
        view = qkv[:, i * h * 128:(i + 1) * h * 128].view(-1, h, 128)
        got = vv.paper_prepare(view, frames=frames, spatial=fh * fw, l2norm=proj == "k",
                               conv=conv, proj=proj, frame_size=(fh, fw))
        ref = vv.paper_prepare(view.contiguous(), frames=frames, spatial=fh * fw,
                               l2norm=proj == "k", conv=conv, proj=proj, frame_size=(fh, fw))
        assert torch.equal(got, ref)


def test_conv_prepare_rejects_bad_geometry(device):
    conv = _sep_conv(2, ("k",), 1).to(device)
    raw = torch.zeros(12, 2, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="frame_size"):
        vv.paper_prepare(raw, frames=2, spatial=6, l2norm=True, conv=conv, proj="k",
                         frame_size=(2, 2))
    wide = _sep_conv(3, ("k",), 1).to(device)
    with pytest.raises(ValueError, match="channels"):
        vv.paper_prepare(raw, frames=2, spatial=6, l2norm=True, conv=wide, proj="k",
                         frame_size=(2, 3))
    # projections the conv does not list take the plain SiLU / L2 path
    plain = vv.paper_prepare(raw, frames=2, spatial=6, l2norm=True, conv=conv, proj="q",
                             frame_size=(2, 3))
    assert torch.equal(plain, vv.paper_prepare(raw, frames=2, spatial=6, l2norm=True))


@pytest.mark.parametrize("projs", [("k", "v"), ("q", "k", "v")])
@pytest.mark.parametrize("text", [False, True])
def test_branch_with_short_conv_against_fp64_oracle(device, projs, text):
    """The VDA body with the short conv on K and V (the released checkpoints) or on all
    three projections, against the float64 oracle with the same convolutions."""
    frames, fh, fw, h = 6, 5, 7, 2
    spatial = fh * fw
    raw, beta, gate, alpha, w, tx = _branch_inputs(frames, spatial, h, 17, text)
    conv = _sep_conv(h, projs, 9)
    weights = {p: _conv_weights(conv, p) for p in projs}
    bounds = ov.window_bounds(frames, 1)
    dev = lambda x: x.to(device)
    out = vv.vda_forward(*map(dev, raw), dev(beta), dev(gate), dev(alpha), bounds, frames, spatial,
                         dev(w), 1e-6, text=None if tx is None else tuple(map(dev, tx)),
                         conv=conv.to(device), frame_size=(fh, fw))
    ref, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6, text=tx,
                             conv=weights, frame_size=(fh, fw))
    close_rel(out, ref, 0.004)


def test_branch_at_production_structure(device):
    """The structure of the released checkpoints' call (configs/training/
    stage_a1_c1_vdn_anchor.yaml): a chunk-aligned window (chunk 3, radius 1), anchor frames
    dense in the softmax branch so the linear branch runs on frames 1 .. F-2 with the bounds
    rebased by -1 (branch.py:380-400), K/V short conv, the text state as a virtual frame and
    boundary chunks of 4 frames (the compose pass), against the float64 oracle."""
    frames, fh, fw, h = 12, 4, 5, 2
    spatial = fh * fw
    lf = frames - 2
    raw, beta, gate, alpha, w, tx = _branch_inputs(lf, spatial, h, 23, text=True)
    bounds = ov.window_bounds(frames, 1, 3)
    lbounds = [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]]
    conv = _sep_conv(h, ("k", "v"), 12)
    weights = {p: _conv_weights(conv, p) for p in ("k", "v")}
    dev = lambda x: x.to(device)
    out = vv.vda_forward(*map(dev, raw), dev(beta), dev(gate), dev(alpha), lbounds, lf, spatial,
                         dev(w), 1e-6, chunk_size=4, text=tuple(map(dev, tx)),
                         conv=conv.to(device), frame_size=(fh, fw))
    ref, _ = ov.paper_branch(*raw, beta, gate, alpha, lbounds, lf, spatial, w, 1e-6, text=tx,
                             chunk_size=4, conv=weights, frame_size=(fh, fw))
    plan = vv.paper_boundary_plan(lbounds, lf, "cpu", 4)
    assert len(plan.cuts) - 1 < lf, "the boundary plan must compose several frames per chunk"
    close_rel(out, ref, 0.004)
