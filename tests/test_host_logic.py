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


def _seven_role_model(device="cpu", blocks=2, k=37, n=21):
    """A model with `blocks` transformer blocks holding one nn.Linear per MXFP8 role at the
    reference's module paths (mxfp8_linear.py:17-25), plus a root Linear and a norm that
    the conversion must leave alone."""
    from torch import nn
    model = nn.Module()
    with torch.device(device):
        model.endpoint = nn.Linear(k, n, dtype=torch.bfloat16)
        model.transformer_blocks = nn.ModuleList()
        for _ in range(blocks):
            block = nn.Module()
            for path in vm.SUPPORTED_ROLES.values():
                parent = block
                *parents, leaf = path.split(".")
                for name in parents:
                    if name not in parent._modules:
                        parent.add_module(name, nn.Module())
                    parent = parent._modules[name]
                parent.add_module(leaf, nn.Linear(k, n, dtype=torch.bfloat16))
            block.norm = nn.LayerNorm(k, dtype=torch.bfloat16)
            model.transformer_blocks.append(block)
    return model.eval().requires_grad_(False)


def test_convert_linear_to_mxfp8_records_meta_symmetry_and_no_device():
    """Default off; enabled, the seven roles of both blocks become MXFP8Linear (14 records),
    the CPU and meta conversions give the same records and state-dict layout, nothing touches
    the GPU, and modules outside the roles keep their parameters
    (tests/test_paper_stack_mxfp8_ops.py:92-110 of the reference states this contract)."""
    from unittest.mock import patch
    cpu, meta = _seven_role_model(), _seven_role_model("meta")
    root, norm = cpu.endpoint.weight, cpu.transformer_blocks[0].norm.weight
    before = root.clone()
    assert vm.convert_linear_to_mxfp8(cpu) == []
    with patch("torch.cuda.init", side_effect=AssertionError("CPU conversion touched the GPU")):
        records = vm.convert_linear_to_mxfp8(cpu, enabled=True, chunk_rows=3)
        assert records == vm.convert_linear_to_mxfp8(meta, enabled=True, chunk_rows=3)
    assert len(records) == 14
    assert {r["role"] for r in records} == set(vm.SUPPORTED_ROLES)
    assert [r["block"] for r in records] == [0] * 7 + [1] * 7
    assert root is cpu.endpoint.weight and norm is cpu.transformer_blocks[0].norm.weight
    assert torch.equal(root, before)
    left, right = cpu.state_dict(), meta.state_dict()
    assert left.keys() == right.keys()
    for key in left:
        assert left[key].shape == right[key].shape and left[key].dtype == right[key].dtype
    packed = cpu.transformer_blocks[0].attn.orig.to_q
    assert isinstance(packed, vm.MXFP8Linear) and not hasattr(packed, "weight")
    assert vm.projection_features(packed) == (37, 21)
    assert set(dict(packed.named_buffers())) == {"weight_data", "weight_scale"}
    assert packed.weight_data.shape == (128, 128) and packed.weight_scale.shape == (512,)


def test_convert_linear_to_mxfp8_refuses_training_tied_and_device_weights():
    model = _seven_role_model(blocks=1)
    with pytest.raises(ValueError, match="booleans"):
        vm.convert_linear_to_mxfp8(model, enabled=1)
    model.train()
    with pytest.raises(ValueError, match="eval model"):
        vm.convert_linear_to_mxfp8(model, enabled=True)
    model.eval()
    block = model.transformer_blocks[0]
    block.attn.orig.to_k.weight = block.attn.orig.to_q.weight
    with pytest.raises(ValueError, match="tied"):
        vm.convert_linear_to_mxfp8(model, enabled=True)
