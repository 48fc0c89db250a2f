"""CPU pins of the MXFP8 oracle and of the product's CPU weight preparation.

The oracle is checked against: the reference tests' known answers
(tests/golden/mxfp8_kat.json), torch's float8_e4m3fn cast over every bf16 bit pattern
times power-of-two scales, the closed form of the E8M0 rule, the swizzle bijection, and
reconstruction bounds. A planted mistake in any of these fails at least one test.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import mxfp8 as om
from vdn_amd import mxfp8 as vm

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "mxfp8_kat.json")))


def all_bf16_values():
    bits = np.arange(65536, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    return v[np.isfinite(v)]


@pytest.mark.parametrize("shift", [-133, -20, -9, -8, -6, 0, 3, 8, 9])
def test_e4m3_encoder_matches_torch_cast_exhaustive(shift):
    v = all_bf16_values().astype(np.float64) * 2.0 ** shift
    v = v[np.abs(v) <= 448].astype(np.float32)
    ours = om.e4m3fn_encode(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_encoder_random_fp32_and_decode_roundtrip():
    rng = np.random.default_rng(5)
    v = (rng.standard_normal(200_000) * np.exp2(rng.integers(-14, 9, 200_000))).astype(np.float32)
    v = v[np.abs(v) <= 448]
    ours = om.e4m3fn_encode(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    codes = np.arange(256, dtype=np.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]
    assert np.array_equal(om.e4m3fn_encode(om.e4m3fn_decode(codes).astype(np.float32)), codes)


def test_e8m0_rule_matches_closed_form():
    rng = np.random.default_rng(7)
    amax = np.concatenate([
        np.abs(all_bf16_values()),
        (rng.random(100_000) * np.exp2(rng.integers(-149, 127, 100_000))).astype(np.float32),
        np.array([0.0, 448.0, 448.0 * (1 + 2 ** -23), 1.75, 1.75 * (1 + 2 ** -23), 2 ** -126,
                  2 ** -149], dtype=np.float32),
    ]).astype(np.float32)
    assert np.array_equal(om.e8m0_exponent(amax), om.e8m0_exponent_closed_form(amax))


def test_reference_scale_kats():
    kat = KAT["e8m0_boundaries"]
    x = np.repeat(np.array(kat["block_values"], dtype=np.float32)[:, None], 32, axis=1)
    codes, natural, _ = om.quantize(x)
    assert natural[:5, 0].tolist() == kat["scale_bytes_first5"]
    assert np.isfinite(om.dequant(codes, natural)).all()
    for i in range(5):
        e = int(natural[i, 0]) - 127
        expect = torch.from_numpy(x[i] * np.float32(2.0 ** -e)).to(torch.float8_e4m3fn)
        assert np.array_equal(codes[i, :32], expect.view(torch.uint8).numpy())
    kat = KAT["e8m0_powers"]
    x = np.concatenate([np.full((2, 32), v, dtype=np.float32) for v in kat["block_values"]], axis=1)
    _, natural, _ = om.quantize(x)
    assert natural[:2, :3].tolist() == [kat["scale_bytes"]] * 2


def test_swizzle_kat_and_bijection():
    kat = KAT["swizzle_map"]
    rows, blocks = kat["rows"], kat["blocks"]
    natural = (np.arange(rows * blocks).reshape(rows, blocks) % 255).astype(np.uint8)
    flat = om.swizzle(natural)
    for row in range(rows):
        for col in range(blocks):
            idx = ((row // 128) * (blocks // 4) + col // 4) * 512
            idx += (row % 32) * 16 + ((row % 128) // 32) * 4 + col % 4
            assert flat[idx] == natural[row, col]
    kat = KAT["swizzle_unique"]
    r, k = kat["rows"], kat["k"]
    rr, cc = np.meshgrid(np.arange(r), np.arange(k // 32), indexing="ij")
    offsets = om.swizzle_offset(rr, cc, k).reshape(-1)
    assert np.array_equal(np.sort(offsets), np.arange(r * k // 32))
    natural = (np.arange(r * (k // 32)) % 251).astype(np.uint8).reshape(r, k // 32)
    assert np.array_equal(om.unswizzle(om.swizzle(natural), r, k), natural)


@pytest.mark.parametrize("shape", KAT["cpu_shapes"]["shapes"])
def test_product_cpu_quantizer_matches_oracle(shape):
    torch.manual_seed(KAT["cpu_shapes"]["seed"])
    x = torch.randn(shape, dtype=torch.bfloat16)
    before = x.clone()
    data, scales = vm.quantize_cpu(x, chunk_rows=7)
    assert torch.equal(x, before)
    codes, natural, flat = om.quantize(x.float().numpy())
    assert np.array_equal(data.numpy(), codes)
    assert np.array_equal(scales.numpy(), flat)
    d1, s1 = vm.quantize_cpu(x, chunk_rows=1)
    assert torch.equal(d1, data) and torch.equal(s1, scales)
    restored = om.dequant(codes, natural)
    r, k = shape
    assert not restored[r:].any() and not restored[:, k:].any()
    if x.numel():
        np.testing.assert_allclose(restored[:r, :k], x.float().numpy(),
                                   rtol=KAT["cpu_shapes"]["rtol"], atol=KAT["cpu_shapes"]["atol"])


def test_quantizer_reconstruction_bound_with_outliers():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x[:, rng.choice(512, 5, replace=False)] *= 20
    x = om.bf16_round(x)
    codes, natural, _ = om.quantize(x)
    dq = om.dequant(codes, natural)[:64, :512]
    amax = np.abs(x.reshape(64, 16, 32)).max(-1).repeat(32, axis=1)
    # E4M3 keeps 3 mantissa bits: relative step 2^-3, half-step error; subnormals 2^-9 * scale.
    assert (np.abs(dq - x) <= amax * 2.0 ** -4 + 1e-30).all()


@pytest.mark.parametrize("value", [float("nan"), float("inf"), -float("inf")])
def test_cpu_quantizer_rejects_nonfinite(value):
    with pytest.raises(ValueError, match="nonfinite"):
        vm.quantize_cpu(torch.tensor([[value]]))


def test_swizzle_helper_matches_oracle():
    natural = torch.from_numpy((np.arange(256 * 12) % 251).astype(np.uint8).reshape(256, 12))
    assert np.array_equal(vm.swizzle_scales(natural).numpy(), om.swizzle(natural.numpy()))


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(100_000) * np.exp2(rng.integers(-30, 30, 100_000))).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(om.bf16_round(v), ref)


def test_gemm_oracle_matches_torch_dequant_matmul():
    torch.manual_seed(42)
    x = torch.randn(17, 31, dtype=torch.bfloat16)
    w = torch.randn(37, 31, dtype=torch.bfloat16) * 0.02
    bias = torch.randn(37, dtype=torch.bfloat16)
    ac, an, _ = om.quantize(x.float().numpy())
    wc, wn, _ = om.quantize(w.float().numpy())
    y = om.gemm(ac, an, wc, wn, 17, 37, bias.float().numpy())
    ref = (torch.from_numpy(om.dequant(ac, an)[:17]).float()
           @ torch.from_numpy(om.dequant(wc, wn)[:37]).float().T).to(torch.bfloat16) + bias
    np.testing.assert_allclose(y, ref.float().numpy(), rtol=1e-2, atol=1e-2)
    # closed form against the unquantized product: block-32 E4M3 error bound
    exact = x.double() @ w.double().T
    assert np.abs(y - bias.float().numpy() - exact.numpy()).max() < 0.05


def test_prenorm_and_activation_oracles_match_torch():
    torch.manual_seed(1)
    x = torch.randn(9, 256, dtype=torch.bfloat16) * 3
    w = torch.rand(256, dtype=torch.bfloat16) + 0.5
    scale = torch.randn(2, 256, dtype=torch.bfloat16) * 0.1
    shift = torch.randn(2, 256, dtype=torch.bfloat16) * 0.1
    idx = torch.tensor([0, 1, 1, 0, 0, 1, 0, 1, 1])
    ours = om.prenorm(x.float().numpy(), w.float().numpy(), 1e-6, scale.float().numpy(),
                      shift.float().numpy(), idx.numpy())
    normed = torch.nn.functional.rms_norm(x.float(), (256,), w.float(), 1e-6)
    ref = (normed * (1 + scale.float()[idx]) + shift.float()[idx]).to(torch.bfloat16).float()
    ulp = bf16_ulps(ours, ref.numpy())
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99
    g = om.gelu_tanh(x.float().numpy())
    gref = torch.nn.functional.gelu(x.float(), approximate="tanh").to(torch.bfloat16).float()
    assert ((bf16_ulps(g, gref.numpy()) <= 1) | (np.abs(g - gref.numpy()) <= 1e-6)).all()
    xs = torch.randn(9, 512, dtype=torch.bfloat16)
    s = om.swiglu(xs.float().numpy())
    a, gg = xs.float().chunk(2, dim=-1)
    sref = (a * torch.nn.functional.silu(gg)).to(torch.bfloat16).float()
    assert bf16_ulps(s, sref.numpy()).max() <= 1


def bf16_ulps(a, b):
    """Distance in bf16 units in the last place between two arrays of bf16 values."""
    ia = (np.asarray(a, dtype=np.float32).view(np.int32) >> 16).astype(np.int64)
    ib = (np.asarray(b, dtype=np.float32).view(np.int32) >> 16).astype(np.int64)
    # map sign-magnitude to a monotonic integer line
    ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)
