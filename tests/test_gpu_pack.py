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


@pytest.mark.parametrize("gated", [False, True])
def test_pack_zero_scale_groups(gated):
    """Groups with a +-0 scale are stored as q = 0 with the nearest nonzero
    scale of the row (previous group first, else next, else 1.0)."""
    n, k, batch = 64, 1024, 2
    g = torch.Generator(DEV).manual_seed(7)
    canon = torch.randint(0, 256, (batch, n, k // 2), dtype=torch.uint8, device=DEV, generator=g)
    scales = (torch.rand((batch, n, k // 128), device=DEV, generator=g) + 0.5).to(torch.bfloat16)
    mask = torch.rand((batch, n, k // 128), device=DEV, generator=g) < 0.3
    scales = torch.where(mask, torch.zeros_like(scales), scales)
    scales[0, 5, :] = 0.0           # a whole row of zero scales -> 1.0
    scales[1, 7, :3] = -0.0         # leading zeros take the next nonzero scale
    packed, ps = ops.pack_int4_g128(canon, scales, gated=gated)
    torch.cuda.synchronize()
    for b in range(batch):
        ref_bytes, ref_sc = np_tile_pack(canon[b].cpu().numpy(), bf16_bits(scales[b]), gated=gated)
        np.testing.assert_array_equal(packed[b].cpu().numpy(), ref_bytes)
        np.testing.assert_array_equal(bf16_bits(ps[b]), ref_sc)
    assert ((bf16_bits(ps) & 0x7FFF) != 0).all()


def test_pack_rejects_bad_shapes():
    canon = torch.zeros((1, 48, 64), dtype=torch.uint8, device=DEV)  # n % 32 != 0
    scales = torch.zeros((1, 48, 1), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.pack_int4_g128(canon, scales)


@pytest.mark.parametrize("n,k,batch", [(64, 1024, 2), (4096, 2048, 1), (32, 128, 3)])
def test_scale_ratios(n, k, batch):
    """Ratios of consecutive group scales over the packed scales: element e
    of group g is s(e of g-1) / s(e of g), fp32 correctly rounded (the same
    IEEE division on the CPU), 0 in group 0; zero-scale groups were replaced
    by the packer, so every ratio is finite.  Scales span 2^-20 .. 2^20."""

    g = torch.Generator(DEV).manual_seed(n + k)
    canon = torch.randint(0, 256, (batch, n, k // 2), dtype=torch.uint8, device=DEV, generator=g)
    expo = torch.randint(-20, 21, (batch, n, k // 128), device=DEV, generator=g).float()
    scales = ((torch.rand((batch, n, k // 128), device=DEV, generator=g) + 0.5) * torch.exp2(expo)).to(torch.bfloat16)
    scales[0, 3, 1:3] = 0.0
    _, ps = ops.pack_int4_g128(canon, scales, gated=n % 64 == 0)
    ratios = ops.pack_int4_ratios(ps, n=n, k=k)
    torch.cuda.synchronize()
    groups = k // 128
    sv = ps.float().cpu().view(batch, n // 32, groups, 32)
    want = torch.zeros_like(sv)
    want[:, :, 1:] = sv[:, :, :-1] / sv[:, :, 1:]
    got = ratios.cpu().view(batch, n // 32, groups, 32)
    assert ratios.dtype == torch.float32 and ratios.shape == ps.shape
    assert torch.isfinite(got).all()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_scale_ratios_follow_in_place_scale_updates():
    """The resident ratios are derived from the scales: after an in-place
    write to w13_s / w2_s (or new scale tensors) ``scale_ratios()`` recomputes
    them into the same tensors, equal to a fresh computation; with the scales
    unchanged it launches nothing and returns the same tensors."""

    from gaiban_lite_amd.synthetic import LayerShape, make_checkpoint_experts
    from gaiban_lite_amd.weights import ResidentInt4MoEWeights

    shape = LayerShape(experts=3, hidden=512, inter=256, topk=2, has_shared=True)
    print("[pack] ratio refresh", flush=True)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(*make_checkpoint_experts(shape, seed=5, device=DEV),
                                                        experts=3, has_shared=True)
    r13, r2 = res.scale_ratios()
    key = res._ratio_key
    assert res.scale_ratios() == (r13, r2) and res._ratio_key == key
    before13, before2 = r13.clone(), r2.clone()
    res.w13_s[1, :4096].mul_(2.5)   # in place: bumps the version counter
    res.w2_s[2].mul_(0.75)
    a13, a2 = res.scale_ratios()
    assert a13 is r13 and a2 is r2
    torch.cuda.synchronize()
    want13 = ops.pack_int4_ratios(res.w13_s, n=2 * shape.inter, k=shape.hidden)
    want2 = ops.pack_int4_ratios(res.w2_s, n=shape.hidden, k=shape.inter)
    assert torch.equal(a13, want13) and torch.equal(a2, want2)
    assert not torch.equal(a13, before13) and not torch.equal(a2, before2)
    # replacing the scale tensor is seen as well
    res.w2_s = res.w2_s.clone() * 2.0
    b13, b2 = res.scale_ratios()
    torch.cuda.synchronize()
    assert b2 is r2 and torch.equal(b2, ops.pack_int4_ratios(res.w2_s, n=shape.hidden, k=shape.inter))
