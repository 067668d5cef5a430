"""Load-time packer: device tiles equal an independent numpy statement of the layout."""

import numpy as np
import pytest
import torch

from gaiban_lite_amd import ops
from helpers import bf16_bits, np_tile_pack

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("n,k,batch", [(32, 128, 1), (64, 256, 3), (512, 1024, 2)])
def test_pack_matches_numpy_layout(n, k, batch, gated):
    g = torch.Generator(DEV).manual_seed(n + k)
    canon = torch.randint(0, 256, (batch, n, k // 2), dtype=torch.uint8, device=DEV, generator=g)
    scales = torch.rand((batch, n, k // 128), device=DEV, generator=g).to(torch.bfloat16)
    packed, ps = ops.pack_int4_g128(canon, scales, gated=gated)
    torch.cuda.synchronize()
    for b in range(batch):
        ref_bytes, ref_sc = np_tile_pack(canon[b].cpu().numpy(), bf16_bits(scales[b]), gated=gated)
        np.testing.assert_array_equal(packed[b].cpu().numpy(), ref_bytes)
        np.testing.assert_array_equal(bf16_bits(ps[b]), ref_sc)


def test_pack_rejects_bad_shapes():
    canon = torch.zeros((1, 48, 64), dtype=torch.uint8, device=DEV)  # n % 32 != 0
    scales = torch.zeros((1, 48, 1), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.pack_int4_g128(canon, scales)
