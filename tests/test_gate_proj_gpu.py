"""GPU parity of the block's gate projection, FrameKDAAlpha and AdaLN kernels
(vdn_gate_projection, vdn_frame_alpha, vdn_adaln_tables) against the oracle: the closed
forms the oracle is pinned by, then random inputs at the oracle's rounding points."""
import numpy as np
import pytest
import torch

from oracle import block as ob
from oracle import mxfp8 as omx
from test_oracle_block import (SMALL, check_adaln_closed_forms, check_alpha_closed_forms,
                               check_gate_closed_forms, oracle_alpha)
from vdn_amd import block as vb
from vdn_amd.block import BlockConfig, BlockWeights

pytestmark = pytest.mark.gpu

WIDE = BlockConfig(hidden=512, heads=40, head_dim=128, ffn=512, context=16, lora_rank=8)
# an odd head count runs the kernel on one zero-padded extra head
ODD = BlockConfig(hidden=320, heads=5, head_dim=128, ffn=384, context=16, lora_rank=8)


def _bf16(x):
    return torch.from_numpy(omx.bf16_round(np.asarray(x, dtype=np.float64)))


def _cuda(tensors):
    return {k: v.cuda() for k, v in tensors.items()}


def kernel_tables(tensors, cfg, temb):
    t = _cuda(tensors)
    tables = vb.adaln_tables(temb.float().cuda(), t["adaln_w"], t["adaln_b"], cfg.hidden)
    return [x.double().cpu() for x in tables]


def kernel_gates(tensors, cfg, x1, frames=1):
    """(soft gate, beta, output gate, gate_down, partial) from the kernel; the output gate is
    formed from the kernel's down projection as the VDA readout forms it."""
    t = _cuda(tensors)
    xg = x1.to(torch.bfloat16).cuda()
    soft, beta, down, partial = vb.gate_projection(
        xg, vb.gate_weight(BlockWeights(t), cfg), t["soft_gate_b"], cfg.heads, frames,
        x1.shape[0] // frames)
    torch.cuda.synchronize()
    d = down.double().cpu()
    up = _bf16((d @ tensors["lgate_up_w"].double().T + tensors["lgate_up_b"].double()).numpy())
    lin = _bf16(torch.sigmoid(up).numpy())
    return soft.double().cpu(), beta.double().cpu(), lin, d, partial.cpu()


def kernel_alpha(tensors, cfg, mean, spatial=200):
    """alpha from the two kernels for x1 whose rows in frame f all equal mean[f] (bf16
    values, so the frame mean is exact); 200 rows make two blocks per frame, one partial."""
    frames = mean.shape[0]
    x1 = mean.repeat_interleave(spatial, dim=0)
    t = _cuda(tensors)
    *_, partial = vb.gate_projection(x1.to(torch.bfloat16).cuda(),
                                     vb.gate_weight(BlockWeights(t), cfg), t["soft_gate_b"],
                                     cfg.heads, frames, spatial)
    alpha = vb.frame_alpha(partial, frames, spatial, t["alpha_up_w"], t["dt_bias"],
                           t["a_log"], cfg.heads, cfg.head_dim)
    return alpha.cpu()


@pytest.fixture(scope="module")
def small():
    return BlockWeights.random(SMALL, seed=5)


@pytest.fixture(scope="module")
def wide():
    return BlockWeights.random(WIDE, seed=6)


@pytest.fixture(scope="module")
def odd():
    return BlockWeights.random(ODD, seed=7)


def test_adaln_closed_forms(small):
    check_adaln_closed_forms(lambda t, temb: kernel_tables(t, SMALL, temb), small, SMALL)


def test_frame_alpha_closed_forms(small):
    check_alpha_closed_forms(lambda t, mean: kernel_alpha(t, SMALL, mean), small, SMALL)


def test_gate_closed_forms(small):
    check_gate_closed_forms(lambda t, x1: kernel_gates(t, SMALL, x1)[:3], small, SMALL)


def _ulps(a, ref):
    """|a - ref| in units of ref's bf16 spacing (ulp of the larger binade for ref = 0)."""
    ref = ref.numpy()
    mag = np.maximum(np.abs(ref), 2.0 ** -126)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    return np.abs(a.numpy() - ref) / ulp


@pytest.mark.parametrize("frames,spatial,width", [(3, 300, "wide"), (2, 128, "wide"),
                                                 (1, 45, "wide"), (2, 200, "odd")])
def test_gate_projection_matches_oracle(wide, odd, frames, spatial, width):
    """40 heads, hidden 512 (and 5 heads, hidden 320: an odd head count): softmax gate, beta
    and the output-gate down projection within one bf16 rounding of the float64 oracle (fp32
    accumulation against float64), the output gate through the same; FrameKDAAlpha from the
    kernel's per-frame sums against the oracle's frame mean of the same x1. Frames of 300 rows
    end in a partial 128-row block."""
    cfg, w = (WIDE, wide) if width == "wide" else (ODD, odd)
    g = torch.Generator().manual_seed(frames * 1000 + spatial)
    x1 = torch.randn(frames * spatial, cfg.hidden, generator=g).to(torch.bfloat16).double()
    soft, beta, lin, down, partial = kernel_gates(w.tensors, cfg, x1, frames)
    o_soft, o_beta, o_lin = ob.BlockOracle(w.tensors, cfg).small_projections(x1)
    o_down = _bf16((x1 @ w.lgate_down_w.double().T).numpy())
    for name, a, ref in (("soft", soft, o_soft), ("beta", beta, o_beta), ("down", down, o_down),
                         ("lin", lin, o_lin)):
        u = _ulps(a, ref)
        assert u.max() <= 1.0, (name, u.max())
        assert (u == 0).mean() >= 0.97, (name, (u == 0).mean())
    # the per-frame sums of x1 @ alpha_down^T, then alpha
    bpf = -(-spatial // 128)
    sums = partial.double().view(frames, bpf, 128).sum(1)
    ref = (x1 @ w.alpha_down_w.double().T).view(frames, spatial, 128).sum(1)
    np.testing.assert_allclose(sums.numpy(), ref.numpy(), rtol=1e-5, atol=1e-4)
    t = _cuda(w.tensors)
    alpha = vb.frame_alpha(partial.cuda(), frames, spatial, t["alpha_up_w"], t["dt_bias"],
                           t["a_log"], cfg.heads, cfg.head_dim).cpu()
    mean = x1.view(frames, spatial, cfg.hidden).mean(1)
    expect = oracle_alpha(w.tensors, cfg, mean).double()
    np.testing.assert_allclose(alpha.double().numpy(), expect.numpy(), rtol=2e-5, atol=1e-7)


@pytest.mark.parametrize("hidden,m,dtype", [(512, 1, torch.float32), (5120, 1, torch.float32),
                                            (520, 3, torch.float32), (512, 2, torch.bfloat16),
                                            (512, 2, torch.float16)])
def test_adaln_tables_match_oracle(hidden, m, dtype):
    """Random temb (m rows, fp32, bf16 or fp16) and weights: every table entry within one bf16
    rounding of the float64 oracle, nearly all equal; K = 520 covers a partial last
    512-column piece. The oracle takes temb.float() (exact for fp16 and bf16), as the
    reference's SiLU(temb.float()) does."""
    g = torch.Generator().manual_seed(hidden + m)
    cfg = BlockConfig(hidden=hidden, heads=4, head_dim=128, ffn=512, context=16, lora_rank=8)
    tensors = {"adaln_w": (torch.randn(6 * hidden, hidden, generator=g) * 0.02).to(torch.bfloat16),
               "adaln_b": (torch.randn(6 * hidden, generator=g) * 0.02).to(torch.bfloat16)}
    temb = torch.randn(m, hidden, generator=g).to(dtype)
    t = _cuda(tensors)
    got = [x.double().cpu() for x in vb.adaln_tables(temb.cuda(), t["adaln_w"], t["adaln_b"],
                                                     hidden)]
    temb = temb.float()
    orc = ob.BlockOracle.__new__(ob.BlockOracle)
    orc.w, orc.cfg = tensors, cfg
    ref = [t.double() for t in orc.tables(temb)]
    for c in range(6):
        assert got[c].shape == (m, hidden)
        u = _ulps(got[c], ref[c])
        assert u.max() <= 1.0, (c, u.max())
        assert (u == 0).mean() >= 0.97, (c, (u == 0).mean())


def test_argument_errors(wide):
    """Wrong dtypes, shapes and host tensors raise before any launch."""
    t = _cuda(wide.tensors)
    wg = vb.gate_weight(BlockWeights(t), WIDE)
    x1 = torch.zeros(2 * 64, WIDE.hidden, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        vb.gate_projection(x1.float(), wg, t["soft_gate_b"], WIDE.heads, 2, 64)
    with pytest.raises(ValueError):
        vb.gate_projection(x1, wg, t["soft_gate_b"], WIDE.heads, 3, 64)   # rows != F * S
    with pytest.raises(ValueError):
        vb.gate_projection(x1, wg[:300], t["soft_gate_b"], WIDE.heads, 2, 64)
    with pytest.raises(ValueError):
        vb.gate_projection(x1.cpu(), wg, t["soft_gate_b"], WIDE.heads, 2, 64)
    *_, partial = vb.gate_projection(x1, wg, t["soft_gate_b"], WIDE.heads, 2, 64)
    with pytest.raises(ValueError):
        vb.frame_alpha(partial, 3, 64, t["alpha_up_w"], t["dt_bias"], t["a_log"], WIDE.heads, 128)
    with pytest.raises(ValueError):
        vb.frame_alpha(partial, 2, 64, t["alpha_up_w"].float(), t["dt_bias"], t["a_log"],
                       WIDE.heads, 128)
    with pytest.raises(ValueError):
        vb.adaln_tables(torch.zeros(1, WIDE.hidden, dtype=torch.int32, device="cuda"),
                        t["adaln_w"], t["adaln_b"], WIDE.hidden)
    with pytest.raises(ValueError):
        vb.adaln_tables(torch.zeros(1, WIDE.hidden, dtype=torch.bfloat16, device="cuda"),
                        t["adaln_w"][:100], t["adaln_b"], WIDE.hidden)
    with pytest.raises(NotImplementedError):
        vb.gate_weight(BlockWeights(t), BlockConfig(hidden=512, heads=80, head_dim=128))
