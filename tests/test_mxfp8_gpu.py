"""GPU parity of the MXFP8 kernels against the oracle (bit-exact codes and scales; GEMM
within the reference's own tolerance rtol .01 / atol .016, test_paper_stack_mxfp8_ops.py:180)."""
import json
import os

import numpy as np
import pytest
import torch
from torch import nn

from oracle import mxfp8 as om
from vdn_amd import mxfp8 as vm

pytestmark = pytest.mark.gpu
KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "mxfp8_kat.json")))


def bf16_ulps(a, b):
    ia = (np.asarray(a, dtype=np.float32).view(np.int32) >> 16).astype(np.int64)
    ib = (np.asarray(b, dtype=np.float32).view(np.int32) >> 16).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


def check_gemm_bound(got, ref, magnitude, ulps=1):
    """|got - ref| <= ulps bf16 ulps + the MFMA accumulation bound times |A||W|^T, and
    nearly all outputs within one bf16 ulp."""
    err = np.abs(got.astype(np.float64) - ref)
    limit = ulps * om.bf16_ulp(ref) + om.MFMA_ACCUMULATION_BOUND * magnitude
    assert (err <= limit).all(), float((err / limit).max())
    assert (bf16_ulps(got, ref) <= 1).mean() > 0.99


def c2_activation(rows, k, seed=0):
    """N(0,1) bf16 activations with 1% of channels scaled x20 (outliers)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g)
    cols = torch.randperm(k, generator=g)[: max(1, k // 100)]
    x[:, cols] *= 20
    return x.to(torch.bfloat16)


def check_quantized(x_cpu, q, s):
    codes, natural, flat = om.quantize(x_cpu.float().numpy())
    assert np.array_equal(q.cpu().numpy(), codes)
    assert np.array_equal(s.cpu().numpy(), flat)


@pytest.mark.parametrize("shape", KAT["cpu_shapes"]["shapes"] + [[300, 5120], [129, 13824]])
def test_quantize_bitexact_small(device, shape):
    torch.manual_seed(13)
    x = torch.randn(shape, dtype=torch.bfloat16) * 3
    q, s = vm.quantize_activation(x.to(device))
    check_quantized(x, q, s)


def test_quantize_strided_and_unaligned_rows(device):
    torch.manual_seed(42)
    base = torch.randn(258, 37, dtype=torch.bfloat16)
    q, s = vm.quantize_activation(base.to(device)[::2])  # row stride 74, K % 8 != 0
    check_quantized(base[::2], q, s)
    base = torch.randn(64, 3 * 256, dtype=torch.bfloat16)
    q, s = vm.quantize_activation(base.to(device)[:, 256:512])  # fused-QKV column slice
    check_quantized(base[:, 256:512], q, s)


def test_quantize_ragged_k_on_a_wider_row(device):
    """K = 520 (a multiple of 8, not of 128) as a view of 1040-wide rows, 200 rows: the last
    128-column chunk holds 8 real columns; the 120 past K must quantize as zero although the
    memory there holds the next columns of the row."""
    torch.manual_seed(7)
    base = torch.randn(200, 1040, dtype=torch.bfloat16) * 5
    view = base.to(device)[:, :520]
    q, s = vm.quantize_activation(view)
    check_quantized(base[:, :520].contiguous(), q, s)


@pytest.mark.parametrize("arrangement", ["sorted", "perm0", "perm1", "perm2"])
def test_quantize_every_bf16_value(device, arrangement):
    """All 63k finite bf16 patterns, packed into blocks two different ways."""
    bits = np.arange(65536, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    vals = vals[np.isfinite(vals)]
    if arrangement != "sorted":
        vals = np.random.default_rng(int(arrangement[-1])).permutation(vals)
    vals = np.concatenate([vals, np.zeros((-len(vals)) % 256, dtype=np.float32)])
    x = torch.from_numpy(vals.reshape(-1, 256)).to(torch.bfloat16)
    q, s = vm.quantize_activation(x.to(device))
    check_quantized(x, q, s)


def test_quantize_c2_shape_sampled_rows(device):
    x = c2_activation(32768, 5120)
    q, s = vm.quantize_activation(x.to(device))
    rows = np.sort(np.random.default_rng(1).choice(32768 // 128, 16, replace=False))
    qc, sc = q.cpu().numpy(), om.unswizzle(s.cpu().numpy(), 32768, 5120)
    for tile in rows:
        sl = slice(tile * 128, tile * 128 + 128)
        codes, natural, _ = om.quantize(x[sl].float().numpy())
        assert np.array_equal(qc[sl], codes)
        assert np.array_equal(sc[sl], natural)


def test_quantize_rejects_nonfinite(device):
    x = torch.ones(3, 64, dtype=torch.bfloat16, device=device)
    x[1, 5] = float("nan")
    with pytest.raises(ValueError, match="nonfinite MXFP8 activation"):
        vm.quantize_activation(x)
    vm.quantize_activation(x, check_finite=False)
    with pytest.raises(ValueError, match="CUDA BF16"):
        vm.quantize_activation(x.float())


@pytest.mark.parametrize("rows,k,weight_f32,tables_f32", [(300, 5120, False, False),
                                                           (37, 256, True, True),
                                                           (5, 1000, False, True),
                                                           (64, 6144, False, False),
                                                           (9, 1001, True, False)])
def test_prenorm_quantize(device, rows, k, weight_f32, tables_f32):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16) * 2
    w = (torch.rand(k, generator=g) + 0.5).to(torch.float32 if weight_f32 else torch.bfloat16)
    tdt = torch.float32 if tables_f32 else torch.bfloat16
    scale = (torch.randn(3, k, generator=g) * 0.2).to(tdt)
    shift = (torch.randn(3, k, generator=g) * 0.2).to(tdt)
    idx = torch.randint(0, 3, (rows,), generator=g)
    y, q, s, finite = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6,
                                                 scale.to(device), shift.to(device),
                                                 idx.to(device), write_bf16=True)
    ref, mag = om.prenorm(x.float().numpy(), w.float().numpy(), 1e-6, scale.float().numpy(),
                          shift.float().numpy(), idx.numpy(), return_magnitude=True)
    yc = y.float().cpu().numpy()
    ulps = bf16_ulps(yc, ref)
    # One fp32 ulp of difference in the row's rsqrt (reduction order) can move the bf16
    # result by one ulp, or by more where the final addition cancels: bound that part by a
    # few fp32 ulps of the addends' magnitude.
    assert ((ulps <= 1) | (np.abs(yc - ref) <= 2.0 ** -21 * mag)).all()
    assert (ulps == 0).mean() > 0.999
    # quantization of the produced bf16 row is bit-exact
    check_quantized(y.cpu(), q, s)
    assert bool(finite.all())
    _, q2, s2, _ = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6, scale.to(device),
                                              shift.to(device), idx.to(device), write_bf16=False)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.parametrize("rows,k,pattern,f32", [(300, 5120, "shared", False),
                                                 (300, 5120, "groups", False),
                                                 (129, 1024, "shared", True),
                                                 (77, 2048, "groups", True),
                                                 (260, 4096, "mixed", False)])
def test_prenorm_quantize_full_rows(device, rows, k, pattern, f32):
    """Row widths of 1024, 2048, 4096 and 5120 columns, whose kernel stages a table row shared
    by a workgroup's rows in LDS: one table row for every row ("shared"), one per 8-row group
    ("groups": each group shared, the groups differing) and per-row indices ("mixed")."""
    g = torch.Generator().manual_seed(k + rows)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16) * 2
    w = (torch.rand(k, generator=g) + 0.5).to(torch.float32 if f32 else torch.bfloat16)
    tdt = torch.float32 if f32 else torch.bfloat16
    scale = (torch.randn(3, k, generator=g) * 0.2).to(tdt)
    shift = (torch.randn(3, k, generator=g) * 0.2).to(tdt)
    if pattern == "shared":
        idx = torch.full((rows,), 2, dtype=torch.long)
    elif pattern == "groups":
        idx = (torch.arange(rows) // 8 + 1) % 3
    else:
        idx = torch.randint(0, 3, (rows,), generator=g)
    y, q, s, finite = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6,
                                                 scale.to(device), shift.to(device),
                                                 idx.to(device), write_bf16=True)
    ref, mag = om.prenorm(x.float().numpy(), w.float().numpy(), 1e-6, scale.float().numpy(),
                          shift.float().numpy(), idx.numpy(), return_magnitude=True)
    yc = y.float().cpu().numpy()
    ulps = bf16_ulps(yc, ref)
    assert ((ulps <= 1) | (np.abs(yc - ref) <= 2.0 ** -21 * mag)).all()
    assert (ulps == 0).mean() > 0.999
    check_quantized(y.cpu(), q, s)
    assert bool(finite.all())
    _, q2, s2, f2 = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6, scale.to(device),
                                               shift.to(device), idx.to(device), write_bf16=False)
    assert torch.equal(q2, q) and torch.equal(s2, s) and torch.equal(f2, finite)


def test_prenorm_full_rows_finite_flags(device):
    x = torch.randn(20, 5120, dtype=torch.bfloat16)
    x[3, 4000] = float("inf")
    x[17, 11] = float("nan")
    w = torch.ones(5120, dtype=torch.bfloat16)
    t = torch.zeros(1, 5120, dtype=torch.bfloat16)
    idx = torch.zeros(20, dtype=torch.long, device=device)
    for write_bf16 in (True, False):
        _, _, _, finite = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6, t.to(device),
                                                     t.to(device), idx, write_bf16=write_bf16)
        assert finite.shape == (128,)
        expect = [True] * 128
        expect[3] = expect[17] = False
        assert finite.cpu().tolist() == expect


def test_prenorm_finite_flags(device):
    x = torch.randn(5, 256, dtype=torch.bfloat16)
    x[2, 7] = float("inf")
    w = torch.ones(256, dtype=torch.bfloat16)
    t = torch.zeros(1, 256, dtype=torch.bfloat16)
    _, _, _, finite = vm.launch_prenorm_quantize(x.to(device), w.to(device), 1e-6, t.to(device),
                                                 t.to(device), torch.zeros(5, dtype=torch.long,
                                                 device=device), write_bf16=False)
    assert finite.shape == (128,)
    assert finite.cpu().tolist() == [True, True, False] + [True] * 125


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_activation_quantize(device, act):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(257, 2 * 1000, generator=g) * 3).to(torch.bfloat16)
    if act == "gelu":
        q, s, finite = vm.launch_gelu_quantize(x.to(device))
        v = om.gelu_tanh(x.float().numpy())
    else:
        q, s, finite = vm.launch_swiglu_quantize(x.to(device))
        v = om.swiglu(x.float().numpy())
    assert bool(finite.all())
    codes, natural, _ = om.quantize(v)
    qc, sc = q.cpu().numpy(), om.unswizzle(s.cpu().numpy(), *codes.shape)
    # the activation's bf16 value may differ by one ulp (transcendental last bits); the
    # quantization of a given bf16 value is exact, so codes agree almost everywhere and
    # the dequantized values within one E4M3 step of the block maximum
    assert (qc == codes).mean() > 0.999 and (sc == natural).mean() > 0.999
    dq, dr = om.dequant(qc, sc), om.dequant(codes, natural)
    amax = np.abs(dr.reshape(dr.shape[0], -1, 32)).max(-1).repeat(32, axis=1)
    assert (np.abs(dq - dr) <= amax * 2.0 ** -3 + 1e-6).all()


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_activation_finite_flags_per_tile(device, act):
    """One finite flag per (16-row, 256-column) output tile, like the reference producer's
    grid (mxfp8_kernels.py:113-124): R = 300 rows (RP 384 -> 24 row tiles), K = 1000 output
    columns (KP 1024 -> 4 column tiles). A nonfinite input clears exactly its tile's flag;
    for SwiGLU both the a and the g half count, and an overflowing a * silu(g) does too."""
    rows, k = 300, 1000
    width = 2 * k if act == "swiglu" else k
    x = torch.ones(rows, width, dtype=torch.bfloat16)
    bad = {(0, 0): float("nan"), (17, 300): float("inf"), (299, 999): -float("inf")}
    if act == "swiglu":
        bad.update({(40, k + 600): float("nan"), (100, 255): 3e38})   # g half; overflow
        x[100, k + 255] = 3e38
    for (r, c), v in bad.items():
        x[r, c] = v
    fn = vm.launch_swiglu_quantize if act == "swiglu" else vm.launch_gelu_quantize
    _, _, finite = fn(x.to(device))
    assert finite.shape == (24 * 4,) and finite.dtype == torch.bool
    expect = torch.ones(24, 4, dtype=torch.bool)
    for r, c in bad:
        expect[r // 16, (c % k if act == "swiglu" else c) // 256] = False
    assert torch.equal(finite.cpu().view(24, 4), expect)


# ---------------------------------------------------------------------------- GEMM ----

@pytest.mark.parametrize("mnk", KAT["gemm_shapes"]["mnk"])
def test_gemm_reference_shapes(device, mnk):
    m, n, k = mnk
    torch.manual_seed(42)
    base = torch.randn(m * 2, k, dtype=torch.bfloat16)
    x = base[::2]
    linear = nn.Linear(k, n, bias=True, dtype=torch.bfloat16).eval()
    packed = vm.MXFP8Linear(linear).to(device)
    y = packed(base.to(device)[::2])
    assert y.shape == (m, n) and y.dtype == torch.bfloat16 and bool(y.isfinite().all())
    if m:
        ac, an, _ = om.quantize(x.float().numpy())
        wc, wn, _ = om.quantize(linear.weight.detach().float().numpy())
        ref = om.gemm(ac, an, wc, wn, m, n, linear.bias.detach().float().numpy())
        np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=KAT["gemm_shapes"]["rtol"],
                                   atol=KAT["gemm_shapes"]["atol"])
    assert torch.equal(packed.weight_data.cpu(), vm.quantize_cpu(linear.weight.detach())[0])


def random_mx(rows, kp, seed, lo=110, hi=140):
    """Random finite E4M3 codes with random per-(row, block) scale bytes."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, size=(rows, kp), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3F
    natural = rng.integers(lo, hi, size=(rows, kp // 32), dtype=np.uint8)
    return codes, natural


@pytest.mark.parametrize("m,n,kp", [(128, 128, 128), (256, 384, 640), (1024, 1024, 512),
                                    (1280, 1152, 384)])
def test_gemm_scale_layout_stress(device, m, n, kp):
    """Independent per-(row, K-block) scales on both operands pin the MFMA lane layout and
    the per-lane E8M0 scale selection."""
    ac, an = random_mx(m, kp, 1)
    wc, wn = random_mx(n, kp, 2)
    a_s, w_s = om.swizzle(an), om.swizzle(wn)
    y = vm.mxfp8_gemm(torch.from_numpy(ac).to(device), torch.from_numpy(a_s).to(device),
                      torch.from_numpy(wc).to(device), torch.from_numpy(w_s).to(device), n)
    ref = om.gemm(ac, an, wc, wn, m, n)
    got = y.float().cpu().numpy()
    check_gemm_bound(got, ref, om.gemm_magnitude(ac, an, wc, wn, m, n))
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=np.abs(ref).max() * 1e-3)


@pytest.mark.parametrize("n", [5120, 15360, 13824])
def test_gemm_c2_shapes_sampled(device, n):
    m, k = 32768, 5120
    x = c2_activation(m, k)
    g = torch.Generator().manual_seed(n)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    q, s = vm.quantize_activation(x.to(device))
    wq, ws = vm.quantize_activation(w.to(device))
    y = vm.mxfp8_gemm(q, s, wq, ws, n, rows=m)
    rows = np.sort(np.random.default_rng(n).choice(m, 256, replace=False))
    ac, an, _ = om.quantize(x[rows].float().numpy())
    wc, wn, _ = om.quantize(w.float().numpy())
    ref = om.gemm(ac, an, wc, wn, len(rows), n)
    got = y[torch.from_numpy(rows).to(device)].float().cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=0.01, atol=0.016)
    check_gemm_bound(got, ref, om.gemm_magnitude(ac, an, wc, wn, len(rows), n))


def test_gemm_accumulate_and_bias(device):
    m, n, k = 300, 384, 256
    torch.manual_seed(5)
    x = torch.randn(m, k, dtype=torch.bfloat16)
    w = torch.randn(n, k, dtype=torch.bfloat16) * 0.05
    bias = torch.randn(n, dtype=torch.bfloat16)
    q, s = vm.quantize_activation(x.to(device))
    wq, ws = vm.quantize_activation(w.to(device))
    base = torch.randn(m, n, dtype=torch.bfloat16)
    out = base.to(device)
    vm.mxfp8_gemm(q, s, wq, ws, n, rows=m, bias=bias.to(device), out=out, accumulate=True)
    ac, an, _ = om.quantize(x.float().numpy())
    wc, wn, _ = om.quantize(w.float().numpy())
    y = om.gemm(ac, an, wc, wn, m, n, bias.float().numpy())
    ref = om.bf16_round(base.float().numpy() + y)
    got = out.float().cpu().numpy()
    # y and y + bias are each rounded to bf16 before the add into `out`: their ulps bound
    # the rounding flips an accumulation error can cause, on top of the final rounding.
    y_raw = om.bf16_round(om.gemm(ac, an, wc, wn, m, n))
    inter = om.bf16_ulp(y_raw) + om.bf16_ulp(y)
    err = np.abs(got.astype(np.float64) - ref)
    limit = inter + om.bf16_ulp(ref) + om.MFMA_ACCUMULATION_BOUND * om.gemm_magnitude(ac, an, wc, wn, m, n)
    assert (err <= limit).all(), float((err / limit).max())
    assert (bf16_ulps(got, ref) == 0).mean() > 0.99


@pytest.mark.parametrize("in_place", [False, True])
def test_gemm_gated_residual_epilogue(device, in_place):
    """out = bf16(res + bf16(gate * bf16(addend + bf16(bf16(acc) + bias)))) with a strided
    residual/addend, optionally written over the residual itself."""
    m, n, k = 260, 384, 512
    g = torch.Generator().manual_seed(21)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    gate = torch.randn(n, generator=g).to(torch.bfloat16)
    wide = torch.randn(m, 2 * n, generator=g).to(torch.bfloat16)
    res, add = wide[:, :n], wide[:, n:]
    q, s = vm.quantize_activation(x.to(device))
    wq, ws = vm.quantize_activation(w.to(device))
    wide_d = wide.to(device)
    res_d, add_d = wide_d[:, :n], wide_d[:, n:]
    out = res_d if in_place else None
    y = vm.mxfp8_gemm(q, s, wq, ws, n, rows=m, bias=bias.to(device), out=out, addend=add_d,
                      residual=res_d, gate=gate.to(device))
    if in_place:
        assert y.data_ptr() == res_d.data_ptr()
    ac, an, _ = om.quantize(x.float().numpy())
    wc, wn, _ = om.quantize(w.float().numpy())
    f = lambda t: t.float().numpy()
    y0 = om.bf16_round(om.gemm(ac, an, wc, wn, m, n))
    y1 = om.bf16_round(y0 + f(bias)[None])
    y2 = om.bf16_round(f(add) + y1)
    gy = om.bf16_round(f(gate)[None] * y2)
    ref = om.bf16_round(f(res) + gy)
    got = y.float().cpu().numpy()
    gabs = np.abs(f(gate))[None]
    mag = om.gemm_magnitude(ac, an, wc, wn, m, n)
    limit = (gabs * (om.bf16_ulp(y0) + om.bf16_ulp(y1) + om.bf16_ulp(y2)
                     + om.MFMA_ACCUMULATION_BOUND * mag) + om.bf16_ulp(gy) + om.bf16_ulp(ref))
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= limit).all(), float((err / limit).max())
    assert (bf16_ulps(got, ref) == 0).mean() > 0.99
    if not in_place:
        assert torch.equal(wide_d.cpu(), wide), "inputs are not modified"


@pytest.mark.parametrize("m,n,k,act", [(300, 384, 256, "gelu_tanh"), (1100, 1408, 512, "gelu_tanh"),
                                       (1100, 1408, 512, None), (129, 200, 128, "gelu_tanh")])
def test_gemm_producer_epilogue_matches_separate_passes(device, m, n, k, act):
    """The fused FFN producer (GEMM + bias -> act -> MXFP8 in the epilogue) writes the same
    bytes as the GEMM's bf16 output fed to the stand-alone producer kernel. Shapes cover both
    tile sizes, rows and columns past a 256 tile, and N not a multiple of 128."""
    g = torch.Generator().manual_seed(m + n)
    x = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16).to(device)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).to(device)
    bias = torch.randn(n, generator=g).to(torch.bfloat16).to(device)
    q, s = vm.quantize_activation(x)
    wq, ws = vm.quantize_activation(w)
    fq, fs = vm.mxfp8_gemm_act_quantize(q, s, wq, ws, n, rows=m, bias=bias, act=act)
    y = vm.mxfp8_gemm(q, s, wq, ws, n, rows=m, bias=bias)
    if act == "gelu_tanh":
        rq, rs, _ = vm.launch_gelu_quantize(y)
    else:
        rq, rs = vm.launch_quantize(y)
    assert fq.shape == rq.shape and fs.shape == rs.shape
    assert torch.equal(fq, rq)
    assert torch.equal(fs, rs)


def test_gemm_epilogue_argument_errors(device):
    q, s = vm.quantize_activation(torch.ones(4, 32, dtype=torch.bfloat16, device=device))
    wq, ws = vm.quantize_activation(torch.ones(8, 32, dtype=torch.bfloat16, device=device))
    gate = torch.ones(8, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="gate needs a residual"):
        vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, gate=gate)
    with pytest.raises(ValueError, match="residual must be"):
        vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, residual=torch.ones(4, 7, dtype=torch.bfloat16,
                                                                    device=device))
    with pytest.raises(ValueError, match="bias must be bf16"):
        vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, bias=torch.ones(8, device=device))
    with pytest.raises(ValueError, match="bias must be bf16"):
        vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, bias=torch.ones(7, dtype=torch.bfloat16,
                                                               device=device))
    with pytest.raises(ValueError, match="scales must hold"):
        vm.mxfp8_gemm(q, s[:-4], wq, ws, 8, rows=4)
    with pytest.raises(ValueError, match="codes must be contiguous uint8"):
        vm.mxfp8_gemm(q.view(torch.int8), s, wq, ws, 8, rows=4)
    store = torch.zeros(5, 8, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="overlaps residual"):
        vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, out=store[1:], residual=store[:4])
    # the same view is allowed: in place over the residual
    vm.mxfp8_gemm(q, s, wq, ws, 8, rows=4, out=store[:4], residual=store[:4])


def test_linear_api_paths_agree(device):
    torch.manual_seed(9)
    x = torch.randn(129, 256, dtype=torch.bfloat16, device=device)
    projections = [vm.MXFP8Linear(nn.Linear(256, 17, bias=False, dtype=torch.bfloat16)).to(device)
                   for _ in range(3)]
    for actual, p in zip(vm.project_qkv(projections, x), projections):
        assert torch.equal(actual, p(x))
    lin = nn.Linear(256, 96, dtype=torch.bfloat16)
    cpu_conv = vm.MXFP8Linear(lin)
    gpu_lin = nn.Linear(256, 96, dtype=torch.bfloat16).to(device)
    gpu_lin.load_state_dict(lin.state_dict())
    gpu_conv = vm.MXFP8Linear(gpu_lin)
    assert torch.equal(gpu_conv.weight_data.cpu(), cpu_conv.weight_data)
    assert torch.equal(gpu_conv.weight_scale.cpu(), cpu_conv.weight_scale)


def test_gemm_reports_nonfinite_result(device):
    p = vm.MXFP8Linear(nn.Linear(32, 16, bias=False, dtype=torch.bfloat16)).to(device)
    x = torch.ones(3, 32, dtype=torch.bfloat16, device=device)
    x[0, 0] = float("nan")
    with pytest.raises(ValueError, match="nonfinite MXFP8 activation"):
        p(x)
    x.fill_(1)
    p.weight_data.fill_(127)  # E4M3 NaN code, a corrupted compressed weight
    with pytest.raises(ValueError, match="nonfinite MXFP8 result"):
        p(x)


@pytest.mark.parametrize("m,f,k", [(1100, 640, 512), (2048, 704, 256), (300, 384, 256),
                                   (1024, 520, 128)])
def test_gemm_swiglu_producer_matches_separate_passes(device, m, f, k):
    """The fused SwiGLU producer (the up projection's a and g halves interleaved in 128-row
    blocks, met in the GEMM epilogue) writes the same bytes as the plain [a | g] GEMM fed to
    the stand-alone SwiGLU producer (tp_ff_forward's two steps). Shapes cover the persistent
    kernel, the small-problem path, a SwiGLU width not a multiple of 128 and rows past a tile."""
    g = torch.Generator().manual_seed(m + f)
    x = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16).to(device)
    w = (torch.randn(2 * f, k, generator=g) * 0.05).to(torch.bfloat16).to(device)
    bias = torch.randn(2 * f, generator=g).to(torch.bfloat16).to(device)
    q, s = vm.quantize_activation(x)
    plain = vm.MXFP8Linear(_as_linear(w, bias)).to(device)
    fused = vm.MXFP8Linear.swiglu_up(_as_linear(w, bias)).to(device)
    fq, fs = fused.forward_act_quantized(q, s, rows=m, act="swiglu")
    y = plain.forward_quantized(q, s, rows=m)
    rq, rs, _ = vm.launch_swiglu_quantize(y)
    assert fq.shape == rq.shape and fs.shape == rs.shape
    assert torch.equal(fq, rq)
    assert torch.equal(fs, rs)
    with pytest.raises(ValueError, match="swiglu_up"):
        plain.forward_act_quantized(q, s, rows=m, act="swiglu")


def _as_linear(w, bias):
    lin = nn.Linear(w.shape[1], w.shape[0], dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w.cpu())
        lin.bias.copy_(bias.cpu())
    return lin
