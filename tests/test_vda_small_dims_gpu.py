"""GPU parity of the VDA branch at head dims below 128: BASELINE config C1 (4 frames x 16x16
tokens, 8 heads, head_dim 64) through the gfx950 kernels, and the per-op paths at d = 16, 32,
64. The kernels run on 128-wide rows with the channels zero-padded; the float64 oracle and the
reference's eager body (branch.py:404-482, delta_rule.py:45-60) run at the true head dim."""
import pytest
import torch
import torch.nn.functional as F

from oracle import vda as ov
from vdn_amd import vda as vv

from test_oracle_vda import c1_inputs

pytestmark = pytest.mark.gpu


def rel_err(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-20)).item()


@torch.no_grad()
@pytest.mark.parametrize("alpha_case", ["ones", "kda"])
def test_c1_branch_on_gpu(device, alpha_case):
    """C1 on the GPU path: the fp32 inputs enter as bf16 (the kernels' activation type).
    Bounds: against the float64 oracle of the bf16 path (same rounding points), relative L2
    4e-3 (the reference's branch-vs-fp64 bound); against the reference's CPU path in fp32 on
    the unrounded inputs, relative L2 1e-2 (the bf16 tolerance of the hot path)."""
    q, k, v, beta, gate, alpha, frames, spatial = c1_inputs(alpha_case)
    bounds = ov.window_bounds(frames, 1)
    w = torch.ones(64)
    raw = [x.bfloat16() for x in (q, k, v)]
    gate16 = gate.bfloat16()
    dev = lambda x: x.to(device)
    out = vv.vda_forward(*map(dev, raw), dev(beta), dev(gate16), dev(alpha), bounds, frames,
                         spatial, dev(w), 1e-6)
    assert out.dtype == torch.bfloat16 and out.shape == (frames * spatial, 8 * 64)
    assert torch.isfinite(out).all()
    ref64, _ = ov.paper_branch(*raw, beta, gate16, alpha, bounds, frames, spatial, w, 1e-6)
    assert rel_err(out, ref64) < 4e-3
    eager = ov.eager_branch_fp32(q, k, v, beta, gate, alpha, bounds, frames, spatial, w)
    assert rel_err(out, eager) < 1e-2


@torch.no_grad()
@pytest.mark.parametrize("d", [16, 32, 64])
@pytest.mark.parametrize("text", [False, True])
def test_small_head_dim_branch_against_fp64_oracle(device, d, text):
    frames, spatial, h, chunk = 9, 21, 3, 4
    g = torch.Generator().manual_seed(d + text)
    raw = [torch.randn(frames * spatial, h, d, generator=g).bfloat16() for _ in range(3)]
    beta = torch.rand(frames * spatial, h, generator=g).bfloat16()
    gate = torch.rand(frames * spatial, h, d, generator=g).bfloat16()
    alpha = torch.rand(frames, h, d, generator=g) * 0.2 + 0.8
    w = torch.rand(d, generator=g) + 0.5
    tx = None
    if text:
        tx = (torch.randn(5, h, d, generator=g).bfloat16(),
              torch.randn(5, h, d, generator=g).bfloat16(),
              torch.rand(5, h, generator=g).bfloat16())
    bounds = ov.window_bounds(frames, 1)
    dev = lambda x: x.to(device)
    out = torch.empty(frames * spatial, h * d, dtype=torch.bfloat16, device=device)
    got = vv.vda_forward(*map(dev, raw), dev(beta), dev(gate), dev(alpha), bounds, frames,
                         spatial, dev(w), 1e-6, chunk_size=chunk, out=out,
                         text=None if tx is None else tuple(map(dev, tx)))
    assert got is out
    ref, _ = ov.paper_branch(*raw, beta, gate, alpha, bounds, frames, spatial, w, 1e-6,
                             text=tx, chunk_size=chunk)
    assert rel_err(out, ref) < 4e-3


@torch.no_grad()
@pytest.mark.parametrize("d", [16, 32, 64])
def test_small_head_dim_ops(device, d):
    """paper_prepare, paper_statistics, the scans, the gather, the readout and the epilogue
    at head dim d against the float64 oracle at the same bounds as their 128-wide tests."""
    frames, spatial, h = 5, 33, 2
    g = torch.Generator().manual_seed(100 + d)
    raw = torch.randn(frames * spatial, h, d, generator=g)
    for dtype, l2 in ((torch.bfloat16, True), (torch.float32, False)):
        x = raw.to(dtype)
        got = vv.paper_prepare(x.to(device), frames=frames, spatial=spatial, l2norm=l2)
        ref = ov.prepare(x, frames, spatial, l2)
        assert got.shape == (frames, h, spatial, d) and got.is_contiguous()
        assert rel_err(got, ref) < (5e-3 if dtype == torch.bfloat16 else 5e-7)

    k = F.normalize(torch.randn(frames, h, spatial, d, generator=g), dim=-1).bfloat16()
    v = torch.randn(frames, h, spatial, d, generator=g).bfloat16()
    beta = torch.rand(frames, h, spatial, generator=g)
    a, b = vv.paper_statistics(k.to(device), v.to(device), beta.to(device))
    ra, rb = ov.statistics(k, v, beta)
    assert a.shape == b.shape == (frames, h, d, d)
    assert rel_err(a, ra) < 5e-7 and rel_err(b, rb) < 1e-4

    # factors stay 128-wide (as the reference's); the scans and gather take d
    alpha = torch.rand(frames, h, d, generator=g) * 0.1 + 0.9
    t, j = ov.factors(ra, rb, alpha)
    t, j = t.float().contiguous(), j.float().contiguous()
    seed = torch.randn(h, d, d, generator=g) * 0.3
    bounds = ov.window_bounds(frames, 1)
    plan = vv.paper_boundary_plan(bounds, frames, device, 2)
    bank = vv.paper_boundary_scan(t.to(device), j.to(device), plan, seed.to(device))
    prefix, suffix = ov.scan(t, j, seed)
    assert bank.shape == (2, plan.chunks, h, d, d)
    torch.testing.assert_close(bank[0].double().cpu(), prefix[torch.tensor(plan.cuts[1:]) - 1],
                               atol=3e-6, rtol=3e-5)
    torch.testing.assert_close(bank[1].double().cpu(), suffix[list(plan.cuts[:-1])],
                               atol=3e-6, rtol=3e-5)
    state = vv.paper_gather(bank, alpha.to(device), plan, seed.to(device), torch.float32)
    expected = ov.gather(prefix, suffix, alpha, bounds, seed)
    assert state.shape == (frames, h, d, d)
    torch.testing.assert_close(state.double().cpu(), expected, atol=4e-6, rtol=5e-5)

    # readout + epilogue (explicit gate), and the epilogue alone
    q = F.normalize(torch.randn(frames, h, spatial, d, generator=g), dim=-1).bfloat16()
    st16 = expected.bfloat16()
    gate = torch.rand(frames * spatial, h, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    got = vv.linear_readout(q.to(device), st16.to(device), w.to(device), gate.to(device), 1e-6,
                            frames, spatial, activate_q=False)
    readout = ov.bf16((q.double() @ st16.double().transpose(-1, -2)).float()).double()
    ref = ov.epilogue(readout, w, gate, 1e-6)
    assert got.shape == (frames * spatial, h * d)
    torch.testing.assert_close(got.cpu().double(), ref, atol=0.0078125, rtol=0.016)
    r = torch.randn(frames, h, spatial, d, generator=g).bfloat16()
    got = vv.vdn_linear_epilogue(r.to(device), w.to(device), gate.to(device), 1e-6)
    torch.testing.assert_close(got.cpu().double(), ov.epilogue(r, w, gate, 1e-6),
                               atol=0.0078125, rtol=0.008)


def test_small_head_dim_rejections(device):
    frames, spatial, h, d = 2, 4, 1, 64
    x = torch.zeros(frames * spatial, h, d, dtype=torch.bfloat16, device=device)
    beta = torch.zeros(frames * spatial, h, dtype=torch.bfloat16, device=device)
    alpha = torch.ones(frames, h, d, device=device)
    w = torch.ones(d, device=device)
    bounds = ov.window_bounds(frames, 1)
    with pytest.raises(ValueError, match="head_dim"):
        vv.vda_forward(x[..., :48], x[..., :48], x[..., :48], beta, x[..., :48], alpha[..., :48],
                       bounds, frames, spatial, w[:48], 1e-6)
    with pytest.raises(ValueError, match="bf16 destination"):
        vv.vda_forward(x, x, x, beta, x, alpha, bounds, frames, spatial, w, 1e-6,
                       out_mxfp8=(None, None, 0))
    with pytest.raises(ValueError, match="share the head dim"):
        vv.vda_forward(x, x, x, beta, x, alpha[..., :32].contiguous(), bounds, frames, spatial,
                       w, 1e-6)
    with pytest.raises(ValueError, match="128"):
        vv.paper_delta_factors(torch.zeros(1, d, d, device=device),
                               torch.zeros(1, d, d, device=device))


class _Branch(torch.nn.Module):
    """The attributes paper_readout reads from the reference's linear branch
    (paper_stack.py:266-318): beta_proj, alpha(frame_mean, heads=), output_gate, norm, bridge,
    paper_vda_chunk_size."""

    def __init__(self, hidden, heads, d, g):
        super().__init__()
        self.heads, self.d = heads, d
        self.beta_proj = torch.nn.Linear(hidden, heads, bias=False)
        self.gate_proj = torch.nn.Linear(hidden, heads * d)
        for p in (self.beta_proj.weight, self.gate_proj.weight, self.gate_proj.bias):
            p.data.copy_(torch.randn(p.shape, generator=g) * 0.05)
        self.decay = torch.rand(heads, d, generator=g) * 0.1 + 0.85
        self.norm = torch.nn.RMSNorm(d, eps=1e-6)
        self.bridge = "alpha"
        self.paper_vda_chunk_size = 2

    def alpha(self, frame_mean, heads=None):
        return self.decay.to(frame_mean.device).expand(frame_mean.shape[0], -1, -1)

    def output_gate(self, xv):
        return torch.sigmoid(self.gate_proj(xv))


@torch.no_grad()
@pytest.mark.parametrize("d", [64, 128])
def test_paper_readout_signature_matches_vda_forward(device, d):
    """paper_readout (the reference's signature) forms beta, alpha and the output gate from
    the branch and runs the same kernels as vda_forward given them: identical bytes."""
    frames, spatial, h, hidden = 5, 12, 2, 96
    g = torch.Generator().manual_seed(d)
    br = _Branch(hidden, h, d, g).to(device).to(torch.bfloat16)
    br.decay = br.decay.float()
    xv = torch.randn(frames * spatial, hidden, generator=g).bfloat16().to(device)
    qkv = [torch.randn(frames * spatial, h, d, generator=g).bfloat16().to(device)
           for _ in range(3)]
    bounds = ov.window_bounds(frames, 1)
    got = vv.paper_readout(br, xv, frames, spatial, bounds, qkv, heads=h)
    beta = torch.sigmoid(br.beta_proj(xv))
    gate = br.output_gate(xv).reshape(-1, h, d)
    alpha = br.decay.to(device).expand(frames, -1, -1).float().contiguous()
    want = vv.vda_forward(*qkv, beta, gate, alpha, bounds, frames, spatial, br.norm.weight, 1e-6,
                          chunk_size=2)
    assert got.shape == (frames * spatial, h * d) and torch.equal(got, want)
