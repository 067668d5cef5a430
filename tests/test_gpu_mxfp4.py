"""MXFP4 routed experts (E2M1 codes, one E8M0 scale per 32 K; the reference's
checkpoint format, ``runtime/dsv4_direct/moe_forward.py:126-155``): the packer
against an independent numpy statement of the tile layout, and the decode and
prefill expert kernels against the fp32 dequant oracle (``dequant_mxfp4`` +
``moe_fp32``) to max_rel and rel_fro <= 1e-2, plus the ``TP4MoE`` drop-in.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    ResidentGateWeights,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    ops,
    route_from_logits,
    synthetic as S,
)
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size
from helpers import DeviceMXFP4Source, assert_moe_close, np_tile_pack_mxfp4, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SMALL = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
_LAYERS: dict = {}


def layer(shape, seed=0, scale_fn=None):
    key = (shape, seed, scale_fn)
    if key not in _LAYERS:
        if len(_LAYERS) >= 2:
            _LAYERS.clear()
            torch.cuda.empty_cache()
        w13, s13, w2, s2 = S.make_checkpoint_experts_mxfp4(shape, seed=seed, device=DEV)
        if scale_fn is not None:
            s13, s2 = scale_fn(s13), scale_fn(s2)
        res = ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts,
                                                              has_shared=shape.has_shared)
        _LAYERS[key] = (res, DeviceMXFP4Source(w13, s13, w2, s2))
    return _LAYERS[key]


def check(shape, t, *, rows=None, block_size=None, clamp=0.0, seed=1, ids=None, scale_fn=None):
    print(f"[mxfp4] E={shape.experts} H={shape.hidden} I={shape.inter} k={shape.topk} T={t} bs={block_size}",
          flush=True)
    res, src = layer(shape, scale_fn=scale_fn)
    x = S.make_hidden(t, shape.hidden, seed=seed, device=DEV)
    r = route_from_logits(S.make_logits(t, shape.experts, seed=seed + 1, device=DEV), topk=shape.topk)
    route_ids = r.routing_ids if ids is None else ids
    bs = block_size or ops.block_size_m(t, shape.topk, shape.experts)
    a = deterministic_moe_align_block_size(route_ids, block_size=bs, num_experts=shape.experts)
    out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.experts_workspace_bytes(t, shape.topk, shape.hidden, shape.inter, shape.has_shared),
                     dtype=torch.uint8, device=DEV)
    ops.experts_mxfp4_into(
        x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, experts=shape.experts,
        inter=shape.inter, has_shared=shape.has_shared, route_weights=r.routing_weights,
        sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
        num_tokens_post_padded=a.num_tokens_post_padded, block_size=bs, clamp_limit=clamp,
        out=out, workspace=ws)
    torch.cuda.synchronize()
    rows = np.arange(t) if rows is None else np.asarray(rows)
    ref = O.moe_fp32(to_np_f32(x), route_ids.cpu().numpy(), r.routing_weights.cpu().numpy(), src,
                     shared_index=shape.experts if shape.has_shared else None, clamp_limit=clamp, rows=rows)
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"T={t} bs={bs}")
    print(f"    {err}", flush=True)


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("n,k,batch", [(32, 128, 1), (64, 256, 3), (512, 1024, 2)])
def test_pack_matches_numpy_layout(n, k, batch, gated):
    g = torch.Generator(DEV).manual_seed(n + k + 5)
    canon = torch.randint(0, 256, (batch, n, k // 2), dtype=torch.uint8, device=DEV, generator=g)
    scales = torch.randint(0, 255, (batch, n, k // 32), dtype=torch.uint8, device=DEV, generator=g)
    packed, ps = ops.pack_mxfp4_g32(canon, scales, gated=gated)
    torch.cuda.synchronize()
    for b in range(batch):
        ref_bytes, ref_sc = np_tile_pack_mxfp4(canon[b].cpu().numpy(), scales[b].cpu().numpy(), gated=gated)
        np.testing.assert_array_equal(packed[b].cpu().numpy(), ref_bytes)
        np.testing.assert_array_equal(ps[b].cpu().numpy(), ref_sc)


@pytest.mark.parametrize("bs", [8, 16, 32, 48, 64])
def test_every_block_size(bs):
    check(SMALL, 200, block_size=bs, seed=5)


@pytest.mark.parametrize("t", [1, 8, 64])
def test_small_decode_and_clamp(t):
    check(SMALL, t, seed=7 + t, clamp=10.0)


def test_e8m0_edge_scales():
    """Scale bytes 0 (2^-127, the E8M0 decode rule of moe_forward.py:115-123),
    100, 127 and 135 mixed within rows."""

    def edges(s):
        table = torch.tensor([0, 100, 127, 135], dtype=torch.uint8, device=DEV)
        g = torch.Generator(DEV).manual_seed(3)
        return table[torch.randint(0, 4, s.shape, device=DEV, generator=g)]

    check(SMALL, 64, seed=9, scale_fn=edges)
    check(SMALL, 200, block_size=64, seed=10, scale_fn=edges)


@pytest.mark.parametrize("t", [1, 64])
def test_flash_decode(t):
    check(S.FLASH, t, rows=np.unique(np.r_[np.arange(min(t, 4)), t - 1]), seed=11 + t, clamp=10.0)


def test_flash_prefill_2048_subset():
    check(S.FLASH, 2048, rows=[0, 1, 1000, 2047], seed=13)


def test_flash_prefill_8192_zipf_subset():
    ids = S.zipf_ids(8192, 256, 6, device=DEV)
    hot = int(torch.argmax(torch.bincount(ids.flatten(), minlength=256)))
    hot_rows = torch.nonzero((ids == hot).any(dim=1)).flatten()[[0, -1]].cpu().numpy()
    check(S.FLASH, 8192, rows=np.r_[0, 4097, 8191, hot_rows], seed=17, ids=ids)


def test_tp4moe_dropin_mxfp4():
    """The drop-in layer with MXFP4 experts: gate GEMM, sqrt-softplus routing
    with bias and route_scale 1.5, clamp 10, staged launch chain."""

    res, src = layer(SMALL)
    g = torch.Generator(DEV).manual_seed(11)
    wg = (torch.randn((SMALL.experts, SMALL.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn((SMALL.experts,), device=DEV, generator=g) * 0.05
    cfg = TP4MoEConfig(hidden_size=SMALL.hidden, intermediate_size=SMALL.inter, experts=SMALL.experts,
                       topk=SMALL.topk, route_scale=1.5, clamp_limit=10.0, score_func="sqrtsoftplus",
                       shared_experts=1)
    moe = TP4MoE(config=cfg, resident=res, gate=ResidentGateWeights(weight=wg, bias=bias), device=DEV,
                 global_row_shapes=[64])
    x = S.make_hidden(64, SMALL.hidden, seed=21, device=DEV).view(1, 64, SMALL.hidden)
    with moe.observe_route_tensors() as seen:
        out, _ = moe(x)
    torch.cuda.synchronize()
    r = seen[0]
    ref_route = O.route_topk(r.gate_logits.cpu().numpy(), SMALL.topk, score_func=O.SCORE_SQRTSOFTPLUS,
                             bias=bias.cpu().numpy(), route_scale=1.5)
    np.testing.assert_array_equal(r.ids.cpu().numpy(), ref_route.ids)
    ref = O.moe_fp32(to_np_f32(x.view(64, -1)), ref_route.ids, ref_route.weights, src,
                     shared_index=SMALL.experts, clamp_limit=10.0)
    assert_moe_close(to_np_f32(out.view(64, -1)), ref, what="TP4MoE mxfp4")
    # the staged and the layer path agree with a direct experts call on the same routing
    assert moe.resident.weight_format == "mxfp4_g32"


@pytest.mark.parametrize("t", [1, 16, 17, 64, 1400])
def test_fused_layer_entry_equals_staged_chain(t):
    """``dsv4moe_layer_mxfp4`` (route [in the prologue for T <= 16], align --
    split over workgroups from 8192 ids -- and the MXFP4 experts in one call)
    gives the staged chain's bits, and its routing equals the oracle's."""

    shape = S.LayerShape(experts=64, hidden=512, inter=512, topk=6, has_shared=True)
    print(f"[mxfp4] fused layer T={t}", flush=True)
    res, src = layer(shape, seed=2)
    g = torch.Generator(DEV).manual_seed(31)
    wg = (torch.randn((shape.experts, shape.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn((shape.experts,), device=DEV, generator=g) * 0.05
    cfg = TP4MoEConfig(hidden_size=shape.hidden, intermediate_size=shape.inter, experts=shape.experts,
                       topk=shape.topk, route_scale=2.5, clamp_limit=10.0, score_func="sqrtsoftplus",
                       shared_experts=1)
    moe = TP4MoE(config=cfg, resident=res, gate=ResidentGateWeights(weight=wg, bias=bias), device=DEV,
                 global_row_shapes=[t])
    x = S.make_hidden(t, shape.hidden, seed=t, device=DEV).view(1, t, shape.hidden)
    lg = S.make_logits(t, shape.experts, seed=t + 5, device=DEV)
    fused = moe.forward_tensor(x, router_logits=lg).clone()
    ids_fused = moe._buffers[(t, 0)].route_ids.clone() if (t, 0) in moe._buffers else None
    staged = moe.forward_tensor(x, router_logits=lg, stage_marker=lambda s: None)
    torch.cuda.synchronize()
    assert torch.equal(fused, staged)
    ref_route = O.route_topk(lg.cpu().numpy(), shape.topk, score_func=O.SCORE_SQRTSOFTPLUS, bias=bias.cpu().numpy(),
                             route_scale=2.5)
    if ids_fused is not None:
        np.testing.assert_array_equal(ids_fused.cpu().numpy(), ref_route.ids)
    rows = np.arange(t) if t <= 64 else np.sort(np.random.default_rng(t).choice(t, 64, replace=False))
    ref = O.moe_fp32(to_np_f32(x.view(t, -1)), ref_route.ids, ref_route.weights, src, shared_index=shape.experts,
                     clamp_limit=10.0, rows=rows)
    assert_moe_close(to_np_f32(fused.view(t, -1))[rows], ref, what=f"fused mxfp4 T={t}")


@pytest.mark.parametrize("t,zipf", [(40, False), (600, False), (300, True)])
def test_paired_8_slot_blocks_equal_16_slot_blocks(t, zipf):
    """MXFP4 decode blocks of 8 slots pair up (two consecutive blocks of one
    expert as one 16-slot item) once the experts average at least 4 slots per
    block: bit-identical to the same routing aligned in blocks of 16, runs
    beyond the 16-block position scan and Zipf routing included, and within
    the bar of the fp32 oracle."""

    print(f"[mxfp4] paired 8-slot blocks T={t} zipf={zipf}", flush=True)
    res, src = layer(SMALL)
    x = S.make_hidden(t, SMALL.hidden, seed=71, device=DEV)
    r = route_from_logits(S.make_logits(t, SMALL.experts, seed=72, device=DEV), topk=SMALL.topk)
    ids = S.zipf_ids(t, SMALL.experts, SMALL.topk, seed=73, device=DEV) if zipf else r.routing_ids
    outs = []
    for bs in (8, 16):
        a = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=SMALL.experts)
        out = torch.empty((t, SMALL.hidden), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(ops.experts_workspace_bytes(t, SMALL.topk, SMALL.hidden, SMALL.inter, True),
                         dtype=torch.uint8, device=DEV)
        ops.experts_mxfp4_into(
            x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, experts=SMALL.experts,
            inter=SMALL.inter, has_shared=True, route_weights=r.routing_weights,
            sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
            num_tokens_post_padded=a.num_tokens_post_padded, block_size=bs, clamp_limit=0.0,
            out=out, workspace=ws)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    rows = np.arange(t) if t <= 64 else np.sort(np.random.default_rng(t).choice(t, 64, replace=False))
    ref = O.moe_fp32(to_np_f32(x), ids.cpu().numpy(), r.routing_weights.cpu().numpy(), src,
                     shared_index=SMALL.experts, rows=rows)
    assert_moe_close(to_np_f32(outs[0])[rows], ref, what=f"mxfp4 paired T={t}")
