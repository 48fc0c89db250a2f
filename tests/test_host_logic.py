"""CPU checks of host-side logic that needs no device: the aliasing rule of the GEMM
wrapper's outputs."""
import pytest
import torch

from vdn_amd import mxfp8 as vm


def test_alias_rule_allows_the_same_view_and_disjoint_interleaved_halves():
    wide = torch.zeros(260, 768, dtype=torch.bfloat16)
    res, add = wide[:, :384], wide[:, 384:]
    vm._check_alias(res, res, 260, 384, "residual")          # in place
    vm._check_alias(res, add, 260, 384, "addend")            # interleaved, no shared element
    other = torch.zeros(260, 384, dtype=torch.bfloat16)
    vm._check_alias(other, res, 260, 384, "residual")        # separate buffers


@pytest.mark.parametrize("shift_rows,shift_cols", [(1, 0), (0, 1), (3, 383), (259, 0)])
def test_alias_rule_rejects_partial_overlap(shift_rows, shift_cols):
    store = torch.zeros(600, 768, dtype=torch.bfloat16)
    a = store[:260, :384]
    b = store[shift_rows:shift_rows + 260, shift_cols:shift_cols + 384]
    with pytest.raises(ValueError, match="overlaps residual"):
        vm._check_alias(a, b, 260, 384, "residual")


def test_alias_rule_with_different_row_strides():
    store = torch.zeros(4096 * 2, dtype=torch.bfloat16)
    a = store[:2048].view(16, 128)             # rows 0..2047, stride 128
    b = store[2048:2048 + 16 * 256].view(16, 256)[:, :128]
    vm._check_alias(a, b, 16, 128, "addend")   # b starts where a ends
    c = store[1920:1920 + 16 * 256].view(16, 256)[:, :128]
    with pytest.raises(ValueError, match="overlaps addend"):
        vm._check_alias(a, c, 16, 128, "addend")
