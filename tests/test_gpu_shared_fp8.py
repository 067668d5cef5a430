"""The shared expert in the checkpoint's FP8 format (E4M3 weights, E8M0
128 x 128 block scales; ``SharedExpertSlice``, ``ops/marlin_moe.py:42-74``),
run as dense W8A16 linears that add into the routed output
(``moe_runtime.py:238-263,1860-1873``).

Checked against the oracle ``shared_fp8_bf16`` (pinned on the CPU to the
reference's torch op order) to max_rel and rel_fro <= 1e-2: the entry point
alone (adding into a given routed output), and ``TP4MoE`` with int4 and MXFP4
routed experts plus the FP8 shared expert, fused and staged chains.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    ResidentFP8SharedExpert,
    ResidentGateWeights,
    ResidentInt4MoEWeights,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    ops,
    synthetic as S,
)
from helpers import DeviceExpertSource, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def make_shared(h, i, seed=0):
    w1, s1 = S.make_fp8_block_linear(i, h, seed=seed + 1, device=DEV, std=0.03)
    w3, s3 = S.make_fp8_block_linear(i, h, seed=seed + 2, device=DEV, std=0.03)
    w2, s2 = S.make_fp8_block_linear(h, i, seed=seed + 3, device=DEV, std=0.03)
    raw = [t.cpu().numpy() for t in (w1, s1, w3, s3, w2, s2)]
    return ResidentFP8SharedExpert.from_checkpoint(w1, s1, w3, s3, w2, s2), raw


@pytest.mark.parametrize("t,h,i", [(1, 512, 256), (64, 512, 256), (300, 512, 384), (64, 4096, 2048)])
def test_shared_fp8_add_entry(t, h, i):
    print(f"[shared fp8] T={t} H={h} I={i}", flush=True)
    sh, raw = make_shared(h, i, seed=t)
    x = S.make_hidden(t, h, seed=t + 7, device=DEV)
    routed = (torch.randn((t, h), device=DEV, generator=torch.Generator(DEV).manual_seed(t)) * 0.1).to(torch.bfloat16)
    ws = torch.empty(ops.shared_fp8_workspace_bytes(t, h, i), dtype=torch.uint8, device=DEV)
    out = routed.clone()
    ops.shared_fp8_add_into(x, sh, clamp_limit=10.0, out=out, workspace=ws)
    zero = torch.zeros_like(routed)
    ops.shared_fp8_add_into(x, sh, clamp_limit=10.0, out=zero, workspace=ws)
    torch.cuda.synchronize()
    shared = O.shared_fp8_bf16(to_np_f32(x), *raw, 10.0)
    assert_moe_close(to_np_f32(zero), shared, what="shared alone")
    want = O.bf16_round(to_np_f32(routed) + shared)
    assert_moe_close(to_np_f32(out), want, what="routed + shared")
    # the add is torch.add of two bf16 tensors: out == bf16(routed + bf16(shared)) exactly
    exact = O.bf16_round(to_np_f32(routed) + to_np_f32(zero))
    np.testing.assert_array_equal(to_np_f32(out), exact)


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
def test_layer_with_fp8_shared_expert(fmt):
    print(f"[shared fp8] layer {fmt}", flush=True)
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=False)
    sh, raw = make_shared(shape.hidden, shape.inter, seed=40)
    if fmt == "int4":
        w = S.make_checkpoint_experts(shape, seed=3, device=DEV)
        res = ResidentInt4MoEWeights.from_checkpoint_layout(*w, experts=shape.experts, has_shared=False,
                                                             shared_fp8=sh)
        src = DeviceExpertSource(*w)
    else:
        w = S.make_checkpoint_experts_mxfp4(shape, seed=3, device=DEV)
        res = ResidentMXFP4MoEWeights.from_checkpoint_layout(*w, experts=shape.experts, has_shared=False,
                                                              shared_fp8=sh)
        src = O.MXFP4ExpertSource(*[t.cpu().numpy() for t in w])
    g = torch.Generator(DEV).manual_seed(11)
    wg = (torch.randn((shape.experts, shape.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    cfg = TP4MoEConfig(hidden_size=shape.hidden, intermediate_size=shape.inter, experts=shape.experts,
                       topk=shape.topk, route_scale=1.5, clamp_limit=10.0, score_func="sigmoid", shared_experts=1)
    layer = TP4MoE(config=cfg, resident=res, gate=ResidentGateWeights(weight=wg), device=DEV,
                   global_row_shapes=[64, 200])
    for t in (64, 200):
        x = S.make_hidden(t, shape.hidden, seed=t, device=DEV).view(1, t, shape.hidden)
        lg = S.make_logits(t, shape.experts, seed=t + 1, device=DEV)
        fused = layer.forward_tensor(x, router_logits=lg)
        staged = layer.forward_tensor(x, router_logits=lg, stage_marker=lambda s: None)
        torch.cuda.synchronize()
        assert torch.equal(fused, staged)
        r = O.route_topk(lg.cpu().numpy(), shape.topk, score_func=O.SCORE_SIGMOID, route_scale=1.5)
        xf = to_np_f32(x.view(t, -1))
        routed = O.bf16_round(O.moe_fp32(xf, r.ids, r.weights, src, shared_index=None, clamp_limit=10.0))
        want = O.bf16_round(routed + O.shared_fp8_bf16(xf, *raw, 10.0))
        assert_moe_close(to_np_f32(fused.view(t, -1)), want, what=f"{fmt} T={t}")


def test_shared_expert_in_both_places_is_rejected():
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    sh, _ = make_shared(shape.hidden, shape.inter)
    w = S.make_checkpoint_experts(shape, seed=3, device=DEV)
    with pytest.raises(ValueError, match="not both"):
        ResidentInt4MoEWeights.from_checkpoint_layout(*w, experts=shape.experts, has_shared=True, shared_fp8=sh)
