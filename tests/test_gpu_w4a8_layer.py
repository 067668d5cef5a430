"""The fused W4A8 layer entries (``dsv4moe_layer_w4a8`` over int4 experts,
``dsv4moe_layer_w4a8_mxfp4`` over MXFP4 experts packed for the W4A8 kernels):
route [inside the prologue for T <= 16], align -- split over workgroups from
8192 route ids -- with x quantised to e4m3 by the alignment launch's other
workgroups, then the W4A8 experts chain.  Each gives the bits of the staged
chain (route, align, the experts entry that quantises x itself) through
``TP4MoE(marlin_input_dtype=float8_e4m3fn)``, and matches the W4A8 oracles on
the oracle's own routing (the reference's W4A8 mode,
runtime/dsv4_direct/moe_runtime.py:207-235,1714-1888)."""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    ResidentGateWeights,
    ResidentInt4MoEWeights,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    synthetic as S,
)
from helpers import DeviceExpertSource, DeviceMXFP4Source, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
FP8 = torch.float8_e4m3fn
SHAPE = S.LayerShape(experts=64, hidden=512, inter=512, topk=6, has_shared=True)
_RES: dict = {}


def resident(fmt):
    if fmt not in _RES:
        if fmt == "int4":
            w = S.make_checkpoint_experts(SHAPE, seed=3, device=DEV)
            res = ResidentInt4MoEWeights.from_checkpoint_layout(*w, experts=SHAPE.experts, has_shared=True,
                                                                 marlin_input_dtype=FP8)
            src = DeviceExpertSource(*w)
        else:
            w = S.make_checkpoint_experts_mxfp4(SHAPE, seed=4, device=DEV)
            res = ResidentMXFP4MoEWeights.from_checkpoint_layout(*w, experts=SHAPE.experts, has_shared=True,
                                                                  marlin_input_dtype=FP8)
            src = DeviceMXFP4Source(*w)
        _RES[fmt] = (res, src)
    return _RES[fmt]


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
@pytest.mark.parametrize("t", [1, 16, 17, 64, 1400])
def test_fused_w4a8_layer_equals_staged_chain(fmt, t):
    print(f"[w4a8 layer] {fmt} T={t}", flush=True)
    res, src = resident(fmt)
    g = torch.Generator(DEV).manual_seed(41)
    wg = (torch.randn((SHAPE.experts, SHAPE.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn((SHAPE.experts,), device=DEV, generator=g) * 0.05
    cfg = TP4MoEConfig(hidden_size=SHAPE.hidden, intermediate_size=SHAPE.inter, experts=SHAPE.experts,
                       topk=SHAPE.topk, route_scale=2.5, clamp_limit=10.0, score_func="sqrtsoftplus",
                       shared_experts=1)
    moe = TP4MoE(config=cfg, resident=res, gate=ResidentGateWeights(weight=wg, bias=bias), device=DEV,
                 global_row_shapes=[t], marlin_input_dtype=FP8)
    x = S.make_hidden(t, SHAPE.hidden, seed=100 + t, device=DEV).view(1, t, SHAPE.hidden)
    lg = S.make_logits(t, SHAPE.experts, seed=200 + t, device=DEV)
    fused = moe.forward_tensor(x, router_logits=lg).clone()
    ids_fused = moe._buffers[(t, 0)].route_ids.clone()
    again = moe.forward_tensor(x, router_logits=lg).clone()
    staged = moe.forward_tensor(x, router_logits=lg, stage_marker=lambda s: None)
    torch.cuda.synchronize()
    assert torch.equal(fused, again)
    assert torch.equal(fused, staged)
    ref_route = O.route_topk(lg.cpu().numpy(), SHAPE.topk, score_func=O.SCORE_SQRTSOFTPLUS,
                             bias=bias.cpu().numpy(), route_scale=2.5)
    np.testing.assert_array_equal(ids_fused.cpu().numpy(), ref_route.ids)
    rows = np.arange(t) if t <= 64 else np.sort(np.random.default_rng(t).choice(t, 48, replace=False))
    oracle = O.moe_w4a8_mxfp4_f32 if fmt == "mxfp4" else O.moe_w4a8_f32
    ref = oracle(to_np_f32(x.view(t, -1)), ref_route.ids, ref_route.weights, src, shared_index=SHAPE.experts,
                 clamp_limit=10.0, rows=rows)
    err = assert_moe_close(to_np_f32(fused.view(t, -1))[rows], ref, what=f"fused w4a8 {fmt} T={t}")
    print(f"    {err}", flush=True)
