"""Checkpoint dequantisers of the ``moe_forward`` module on the HIP kernels
(reference ``runtime/dsv4_direct/moe_forward.py:115-176``).

Every output is compared bit for bit (fp32 bit patterns, NaN included) with
an independent CPU computation: torch's own E8M0 and E4M3FN conversions times
the block scale, and the oracle's table-lookup MXFP4 dequantiser (itself
pinned against the numpy oracle).  Shapes cover the vector and the scalar
paths (columns a multiple of 4 or not), rows and columns that are not
multiples of 128, both code dtypes, decoded float scales and the reserved
E8M0 byte 255 (NaN).
"""

import pytest
import torch

import oracle.torch_path as TP
from gaiban_lite_amd import moe_forward as MF

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def bits_equal(got: torch.Tensor, want: torch.Tensor) -> bool:
    got, want = got.cpu(), want.cpu()
    nan_g, nan_w = torch.isnan(got), torch.isnan(want)
    if not torch.equal(nan_g, nan_w):
        return False
    return torch.equal(got[~nan_g].view(torch.int32), want[~nan_w].view(torch.int32))


def test_decode_e8m0_every_code():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e8m0fnu).float()
    for scale in (codes.to(DEV), codes.view(torch.float8_e8m0fnu).to(DEV)):
        got = MF._decoded_e8m0(scale)
        assert got.dtype == torch.float32 and bits_equal(got, want)
    f = torch.randn(7, 3, device=DEV, dtype=torch.bfloat16)
    assert torch.equal(MF._decoded_e8m0(f), f.float())


@pytest.mark.parametrize("rows,k", [(1, 32), (64, 4096), (2048, 512), (37, 96)])
@pytest.mark.parametrize("packed_dtype", [torch.uint8, torch.int8])
def test_dequant_mxfp4_bits(rows, k, packed_dtype):
    print(f"[dequant] mxfp4 rows={rows} k={k} {packed_dtype}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + k)
    packed = torch.randint(0, 256, (rows, k // 2), generator=g, dtype=torch.uint8)
    codes = torch.randint(100, 150, (rows, k // 32), generator=g, dtype=torch.uint8)
    codes[0, 0] = 0  # 2^-127: products become fp32 subnormals
    want = TP.dequant_mxfp4(packed, codes, dtype=torch.float32)
    got = MF.dequant_mxfp4(packed.view(packed_dtype).to(DEV), codes.view(torch.float8_e8m0fnu).to(DEV))
    assert got.shape == (rows, k) and bits_equal(got, want)
    # decoded float scales (any value): the same fp32 products
    fscale = torch.randn((rows, k // 32), generator=g)
    want_f = TP.dequant_mxfp4(packed, torch.zeros_like(codes) + 127, dtype=torch.float32) * \
        fscale.repeat_interleave(32, dim=1)
    assert bits_equal(MF.dequant_mxfp4(packed.to(DEV), fscale.to(DEV)), want_f)


def test_dequant_mxfp4_reserved_scale_is_nan():
    packed = torch.full((4, 64), 0x21, dtype=torch.uint8)
    codes = torch.full((4, 4), 127, dtype=torch.uint8)
    codes[2, 1] = 255
    got = MF.dequant_mxfp4(packed.to(DEV), codes.to(DEV)).cpu()
    nan = torch.zeros((4, 128), dtype=torch.bool)
    nan[2, 32:64] = True
    assert torch.equal(torch.isnan(got), nan)


@pytest.mark.parametrize("rows,cols", [(1, 128), (300, 520), (130, 131), (256, 7168), (4096, 2048)])
@pytest.mark.parametrize("wdtype", [torch.float8_e4m3fn, torch.bfloat16, torch.float16, torch.float32])
def test_dequant_fp8_block_bits(rows, cols, wdtype):
    print(f"[dequant] fp8_block rows={rows} cols={cols} {wdtype}", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    if wdtype == torch.float8_e4m3fn:
        w = torch.randint(0, 256, (rows, cols), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
    else:
        w = (torch.randn((rows, cols), generator=g) * 3).to(wdtype)
    sb = (-(-rows // 128), -(-cols // 128))
    codes = torch.randint(110, 140, sb, generator=g, dtype=torch.uint8)
    codes[0, 0] = 0
    if sb[1] > 1:
        codes[-1, 1] = 255
    scale = codes.view(torch.float8_e8m0fnu).float()
    want = w.float() * scale.repeat_interleave(128, 0).repeat_interleave(128, 1)[:rows, :cols]
    got = MF.dequant_fp8_block(w.to(DEV), codes.view(torch.float8_e8m0fnu).to(DEV))
    assert got.shape == (rows, cols) and bits_equal(got, want)
    # already decoded scales give the same bits
    assert bits_equal(MF.dequant_fp8_block(w.to(DEV), scale.to(DEV)), want)


def test_dequant_of_an_offset_view():
    """A view that starts off the kernels' 16-byte alignment is copied first."""

    g = torch.Generator().manual_seed(5)
    flat = torch.randint(0, 256, (1 + 2 * 64,), generator=g, dtype=torch.uint8)
    packed = flat[1:].view(2, 64)
    codes = torch.full((2, 4), 127, dtype=torch.uint8)
    view = flat.to(DEV)[1:].view(2, 64)
    assert view.data_ptr() % 16 != 0
    assert bits_equal(MF.dequant_mxfp4(view, codes.to(DEV)), TP.dequant_mxfp4(packed, codes))
