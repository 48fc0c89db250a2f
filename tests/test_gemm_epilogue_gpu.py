"""The block-scaled GEMM's fused epilogues at the sizes the 108k block runs them.

Padded M and N >= 1024 select the persistent kernel (bias, gated residual, written out of
place or over the residual) or, for an addend or rows not 16-byte aligned, the 256 x 256
tile kernel. The block's [O | O_lin] GEMM (K = 10240) and FFN-down (K = 13824) run the
gated residual in place over the hidden state; cross-O runs the residual without a gate.

Two checks per case:
  * bit-exact: the same kernel's plain output (bias only; the main loop and so the fp32
    accumulators are identical) carried through the epilogue chain in torch fp32 with one
    bf16 rounding per step: bf16(res + bf16(gate * bf16(addend + y))), y = bf16(bf16(acc) + b);
  * oracle: sampled rows (every 256-row tile edge and the last rows) against the oracle's
    exactly dequantized float64 GEMM and the same chain, within the accumulation bound of
    tests/test_mxfp8_gpu.py::test_gemm_gated_residual_epilogue.
"""
import functools

import numpy as np
import pytest
import torch

from oracle import mxfp8 as om
from vdn_amd import mxfp8 as vm

pytestmark = pytest.mark.gpu

M, N = 2300, 5120          # padded M 2304 = 9 row tiles of 256, the last one partly past M
SENTINEL = 7.0


@functools.lru_cache(maxsize=None)
def operands(k):
    g = torch.Generator().manual_seed(k)
    x = torch.randn(M, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, k, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16)
    gate = torch.randn(N, generator=g).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    add = torch.randn(M, N, generator=g).to(torch.bfloat16)
    rows = np.unique(np.concatenate([np.arange(0, M, 256), np.arange(255, M, 256),
                                     np.arange(M - 4, M),
                                     np.random.default_rng(k).choice(M, 64, replace=False)]))
    wc, wn, _ = om.quantize(w.float().numpy())
    ac, an, _ = om.quantize(x[torch.from_numpy(rows)].float().numpy())
    y0 = om.bf16_round(om.gemm(ac, an, wc, wn, len(rows), N))
    mag = om.gemm_magnitude(ac, an, wc, wn, len(rows), N)
    return dict(x=x, w=w, bias=bias, gate=gate, res=res, add=add, rows=rows, y0=y0, mag=mag)


def bf(t):
    return t.to(torch.bfloat16)


def chain(y, addend=None, residual=None, gate=None):
    """The epilogue's steps after bias in torch fp32, one bf16 rounding each."""
    if addend is not None:
        y = bf(addend.float() + y.float())
    if residual is not None:
        if gate is not None:
            y = bf(gate.float()[None] * y.float())
        y = bf(residual.float() + y.float())
    return y


def oracle_check(op, got, addend, residual, gate):
    """Sampled rows of `got` against the oracle's float64 GEMM and the epilogue chain."""
    rows = op["rows"]
    f = lambda t: None if t is None else t.float().numpy()
    y0 = op["y0"]
    y1 = om.bf16_round(y0 + f(op["bias"])[None])
    ref, limit = y1, om.bf16_ulp(y0) + om.bf16_ulp(y1) + om.MFMA_ACCUMULATION_BOUND * op["mag"]
    if addend is not None:
        ref = om.bf16_round(f(addend)[rows] + ref)
        limit = limit + om.bf16_ulp(ref)
    if residual is not None:
        if gate is not None:
            gy = om.bf16_round(f(gate)[None] * ref)
            limit = np.abs(f(gate))[None] * limit + om.bf16_ulp(gy)
            ref = gy
        ref = om.bf16_round(f(residual)[rows] + ref)
        limit = limit + om.bf16_ulp(ref)
    got = got[torch.from_numpy(rows).to(got.device)].float().cpu().numpy()
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= limit).all(), float((err / limit).max())
    exact = (om.bf16_bits(got) == om.bf16_bits(ref)).mean()
    assert exact > 0.99, exact


def quantized(op, device):
    q, s = vm.quantize_activation(op["x"].to(device))
    wq, ws = vm.quantize_activation(op["w"].to(device))
    return q, s, wq, ws


@pytest.mark.parametrize("k", [10240, 13824])
@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("with_gate", [True, False])
def test_persistent_residual_epilogue(device, k, in_place, with_gate):
    """The persistent kernel's residual epilogue (residual rows prefetched one 16-row group
    ahead), with and without the gate, out of place and over the residual itself. Rows of
    the buffer past M are never written."""
    op = operands(k)
    q, s, wq, ws = quantized(op, device)
    bias, gate = op["bias"].to(device), op["gate"].to(device) if with_gate else None
    plain = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias)
    store = torch.full((M + 9, N), SENTINEL, dtype=torch.bfloat16, device=device)
    store[:M] = op["res"].to(device)
    res = store[:M]
    if in_place:
        out = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, out=res, residual=res, gate=gate)
        assert out.data_ptr() == res.data_ptr()
    else:
        out = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, residual=res, gate=gate)
        assert torch.equal(res, op["res"].to(device)), "the residual input is not modified"
    torch.cuda.synchronize()
    assert bool((store[M:] == SENTINEL).all()), "rows past M are not written"
    expect = chain(plain, residual=op["res"].to(device), gate=gate)
    assert torch.equal(out, expect)
    oracle_check(op, out, None, op["res"], op["gate"] if with_gate else None)


@pytest.mark.parametrize("k", [10240, 13824])
def test_tile_kernel_addend_and_gated_residual(device, k):
    """An addend at M, N >= 1024 takes the 256 x 256 tile kernel: `out += linear(x)`
    (accumulate) and the full chain addend + gated residual, in place over the residual."""
    op = operands(k)
    q, s, wq, ws = quantized(op, device)
    bias, gate = op["bias"].to(device), op["gate"].to(device)
    zeros = torch.zeros(M, N, dtype=torch.bfloat16, device=device)
    plain = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, addend=zeros)   # same kernel
    acc = op["add"].to(device)
    vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, out=acc, accumulate=True)
    assert torch.equal(acc, chain(plain, addend=op["add"].to(device)))
    oracle_check(op, acc, op["add"], None, None)
    res = op["res"].to(device)
    add = op["add"].to(device)
    out = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, out=res, addend=add, residual=res,
                        gate=gate)
    assert torch.equal(out, chain(plain, addend=add, residual=op["res"].to(device), gate=gate))
    oracle_check(op, out, op["add"], op["res"], op["gate"])


def test_tile_kernel_unaligned_rows(device):
    """Output and residual rows not 16-byte aligned (row stride N + 1) take the tile
    kernel's element-wise epilogue."""
    k = 10240
    op = operands(k)
    q, s, wq, ws = quantized(op, device)
    bias, gate = op["bias"].to(device), op["gate"].to(device)
    wide = torch.empty(M, N + 1, dtype=torch.bfloat16, device=device)
    plain = wide[:, :N]
    vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, out=plain)
    resw = torch.empty(M, N + 1, dtype=torch.bfloat16, device=device)
    resw[:, N] = SENTINEL
    resw[:, :N] = op["res"].to(device)
    res = resw[:, :N]
    out = vm.mxfp8_gemm(q, s, wq, ws, N, rows=M, bias=bias, out=res, residual=res, gate=gate)
    assert out.data_ptr() == res.data_ptr()
    assert bool((resw[:, N] == SENTINEL).all()), "the column past N is not written"
    assert torch.equal(out, chain(plain, residual=op["res"].to(device), gate=gate))
    oracle_check(op, out, None, op["res"], op["gate"])
