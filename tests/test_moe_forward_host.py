"""Host-side contracts of the ``moe_forward`` dequantisers
(``runtime/dsv4_direct/moe_forward.py:115-176``): the exception class of each
malformed argument, checked on the CPU before anything is launched, and that
the kernels are never replaced by a CPU computation."""

import pytest
import torch

from gaiban_lite_amd import moe_forward as MF


def test_exports():
    for name in ("dequant_mxfp4", "dequant_fp8_block", "FP4_VALUES", "E8M0"):
        assert name in MF.__all__
    assert MF.E8M0 is torch.float8_e8m0fnu


def test_decoded_e8m0_contract():
    f = torch.randn(3, 4)
    assert torch.equal(MF._decoded_e8m0(f.half()), f.half().float())
    with pytest.raises(TypeError):
        MF._decoded_e8m0(torch.zeros(3, dtype=torch.int32))
    with pytest.raises(TypeError):
        MF._decoded_e8m0([1, 2])
    with pytest.raises(ValueError, match="GPU"):
        MF._decoded_e8m0(torch.zeros(3, dtype=torch.uint8))


def test_dequant_mxfp4_contract():
    packed = torch.zeros((4, 64), dtype=torch.uint8)
    scale = torch.zeros((4, 4), dtype=torch.uint8)
    with pytest.raises(ValueError):
        MF.dequant_mxfp4(packed.view(-1), scale)
    with pytest.raises(ValueError):
        MF.dequant_mxfp4(packed, scale.view(-1))
    with pytest.raises(TypeError):
        MF.dequant_mxfp4(packed.to(torch.int16), scale)
    with pytest.raises(ValueError, match="multiple of the 32-wide"):
        MF.dequant_mxfp4(torch.zeros((4, 24), dtype=torch.uint8), torch.zeros((4, 1), dtype=torch.uint8))
    with pytest.raises(ValueError, match=r"shape \(4, 3\)"):
        MF.dequant_mxfp4(packed, torch.zeros((4, 3), dtype=torch.uint8))
    with pytest.raises(ValueError, match="runs on the GPU"):
        MF.dequant_mxfp4(packed, scale)


def test_dequant_fp8_block_contract():
    w = torch.zeros((130, 300), dtype=torch.float8_e4m3fn)
    scale = torch.zeros((2, 3), dtype=torch.uint8)
    with pytest.raises(ValueError):
        MF.dequant_fp8_block(w.view(-1), scale)
    with pytest.raises(ValueError, match=r"expected \(2, 3\)"):
        MF.dequant_fp8_block(w, torch.zeros((1, 3), dtype=torch.uint8))
    with pytest.raises(TypeError):
        MF.dequant_fp8_block(torch.zeros((130, 300), dtype=torch.int32), scale)
    with pytest.raises(ValueError, match="runs on the GPU"):
        MF.dequant_fp8_block(w, scale)
