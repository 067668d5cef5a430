"""Graph capture of the decode layer call (the reference captures whole decode
stages, ``stateful_graph.py:398-470``, after resetting each MoE slot's
completion event, ``moe_runtime.py:1285-1316``).

``TP4MoE.forward_tensor`` is captured with ``torch.cuda.graph`` (a HIP graph)
and replayed several times with new inputs copied into the captured input
tensors, with eager work and synchronisations between the replays; every
replay must equal an eager call on another slot bit for bit.  The path records
no memset nodes: every launch in it is a kernel, plus the output copy.
"""

import pytest
import torch

from gaiban_lite_amd import ResidentGateWeights, ResidentInt4MoEWeights, TP4MoE, TP4MoEConfig, synthetic as S

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def build(shape, rows):
    w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=9, device=DEV)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts, has_shared=True)
    g = torch.Generator(DEV).manual_seed(21)
    wg = (torch.randn((shape.experts, shape.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn((shape.experts,), device=DEV, generator=g) * 0.05
    cfg = TP4MoEConfig(hidden_size=shape.hidden, intermediate_size=shape.inter, experts=shape.experts,
                       topk=shape.topk, route_scale=2.5, clamp_limit=10.0, score_func="sqrtsoftplus",
                       shared_experts=1)
    return TP4MoE(config=cfg, resident=res, gate=ResidentGateWeights(weight=wg, bias=bias), device=DEV,
                  global_row_shapes=rows, slots_per_shape=2)


@pytest.mark.parametrize("use_logits", [False, True])
@pytest.mark.parametrize("shape,rows", [
    (S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True), 1),
    (S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True), 64),
    (S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True), 8),
    (S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True), 64),
    # 8400 route ids: the workgroup-split alignment (scratch in the workspace)
    (S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True), 1400),
])
def test_capture_and_replay_matches_eager(shape, rows, use_logits):
    print(f"[graph] E={shape.experts} T={rows} logits={use_logits}", flush=True)
    layer = build(shape, [rows])
    xs = [S.make_hidden(rows, shape.hidden, seed=40 + i, device=DEV).view(1, rows, shape.hidden) for i in range(5)]
    lgs = [S.make_logits(rows, shape.experts, seed=60 + i, device=DEV) for i in range(5)]
    x_s = xs[0].clone()
    lg_s = lgs[0].clone()

    def call(x, lg, slot):
        return layer.forward_tensor(x, router_logits=lg if use_logits else None, slot=slot)

    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        for _ in range(3):
            call(x_s, lg_s, 0)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()

    layer.reset_free_slot_completion_event(rows, 0)
    assert layer.slot_completion_status(rows, 0) == {"state": "free", "has_completion_event": False}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = call(x_s, lg_s, 0)
    torch.cuda.synchronize()

    for i in range(1, 5):
        x_s.copy_(xs[i])
        lg_s.copy_(lgs[i])
        graph.replay()
        torch.cuda.synchronize()
        eager = call(xs[i], lgs[i], 1)  # eager work between the replays, other slot
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager), f"replay {i} differs from the eager call"
    # the first input again, after the others
    x_s.copy_(xs[0])
    lg_s.copy_(lgs[0])
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_s, call(xs[0], lgs[0], 1))
    assert layer.slot_completion_status(rows, 0)["state"] == "free"
    del graph
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows", [8, 64])
def test_route_capture_inside_a_bound_graph(rows):
    """The reference's capture protocol (``moe_runtime.py:825-978,1017-1227``):
    register the route capture, reset the slot's completion event, capture the
    call inside ``bind_alignment_provider_for_capture(None, ...)``, reset the
    generation after warm-up, replay with new inputs; each replay writes the
    effective route into the capture buffer and adds one to the device
    generation, and ``snapshot_route_capture`` returns it -- equal to the
    route of an eager call of the same input, and the output equal too."""

    import oracle as O

    shape = S.LayerShape(experts=64, hidden=512, inter=512, topk=6, has_shared=True)
    print(f"[graph] route capture T={rows}", flush=True)
    layer = build(shape, [rows])
    cap = layer.register_route_capture(rows, 0)
    xs = [S.make_hidden(rows, shape.hidden, seed=80 + i, device=DEV).view(1, rows, shape.hidden) for i in range(4)]
    lgs = [S.make_logits(rows, shape.experts, seed=90 + i, device=DEV) for i in range(4)]
    x_s, lg_s = xs[0].clone(), lgs[0].clone()
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        for _ in range(2):
            layer.forward_tensor(x_s, router_logits=lg_s, slot=0)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    assert int(cap.generation.item()) == 2
    layer.reset_free_slot_completion_event(rows, 0)
    graph = torch.cuda.CUDAGraph()
    with layer.bind_alignment_provider_for_capture(None, buffer_keys=[(rows, 0)]):
        with torch.cuda.graph(graph):
            out_s = layer.forward_tensor(x_s, router_logits=lg_s, slot=0)
    torch.cuda.synchronize()
    layer.reset_route_capture_generation(rows, 0)
    for i in range(1, 4):
        x_s.copy_(xs[i])
        lg_s.copy_(lgs[i])
        graph.replay()
        torch.cuda.synchronize()
        ev = layer.snapshot_route_capture(rows, 0, expected_generation=i)
        ref = O.route_topk(lgs[i].cpu().numpy(), shape.topk, score_func=O.SCORE_SQRTSOFTPLUS,
                           bias=layer.gate.bias.cpu().numpy(), route_scale=2.5)
        assert torch.equal(ev.ids, torch.from_numpy(ref.ids))
        assert torch.equal(ev.weights, torch.from_numpy(ref.weights))
        eager = layer.forward_tensor(xs[i], router_logits=lgs[i], slot=1)
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager), f"replay {i} differs from the eager call"
    del graph
    torch.cuda.synchronize()


def test_fixed_b240_provider_layout_eager_and_captured():
    """The fixed B240 provider (``fixed_moe_align.py:67-155,407-421``): its
    layout equals the oracle's brute force for uniform and skewed [240, 6]
    routes (an expert with more than one block, unused experts); a layer
    that aligns through it gives the same bits as the built-in alignment;
    captured inside ``bind_alignment_provider_for_capture(provider, ...)``
    and replayed with new inputs it equals eager calls."""

    import numpy as np

    import oracle as O
    from gaiban_lite_amd import fixed_moe_align as FA

    print("[graph] fixed B240 provider", flush=True)
    g = torch.Generator(DEV).manual_seed(240)
    prov = FA.FixedB240MoEAlignmentProvider(device=DEV, global_row_shapes=(240,), slots_per_shape=2,
                                            route_kind="learned")
    uniform = torch.argsort(torch.rand((240, 256), device=DEV, generator=g), dim=1)[:, :6].to(torch.int32)
    skewed = uniform.clone()
    skewed[:, 0] = 7  # expert 7 in every row: 240 routes = 30 blocks
    skewed[:40, 1] = 3
    skewed = torch.where((skewed == 7) & (torch.arange(6, device=DEV) > 0), torch.full_like(skewed, 11), skewed)
    for ids in (uniform, skewed):
        out, _ = FA.allocate_fixed_b240_alignment(ids)
        got = prov(ids, block_size=8, num_experts=256, output=out, slot=0)
        assert got is out
        torch.cuda.synchronize()
        ref = O.moe_align_bruteforce(ids.cpu().numpy(), 8, 256)
        np.testing.assert_array_equal(out.sorted_token_ids.cpu().numpy(), ref.sorted_token_ids)
        np.testing.assert_array_equal(out.expert_ids.cpu().numpy(), ref.expert_ids)
        assert int(out.num_tokens_post_padded.item()) == ref.num_tokens_post_padded

    shape = S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True)
    base = build(shape, [240])
    layer = TP4MoE(config=base.config, resident=base.resident, gate=base.gate, device=DEV,
                   global_row_shapes=[240], slots_per_shape=2, alignment_provider=prov)
    xs = [S.make_hidden(240, shape.hidden, seed=300 + i, device=DEV).view(1, 240, shape.hidden) for i in range(4)]
    for x in xs[:2]:
        a = layer.forward_tensor(x, slot=1)
        b = base.forward_tensor(x, slot=1)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    x_s = xs[0].clone()
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        for _ in range(2):
            layer.forward_tensor(x_s, slot=0)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    layer.reset_free_slot_completion_event(240, 0)
    graph = torch.cuda.CUDAGraph()
    with layer.bind_alignment_provider_for_capture(prov, buffer_keys=[(240, 0)]):
        with torch.cuda.graph(graph):
            out_s = layer.forward_tensor(x_s, slot=0)
    torch.cuda.synchronize()
    for i in (1, 2, 3, 0):
        x_s.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        eager = base.forward_tensor(xs[i], slot=1)
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager), f"replay of input {i} differs from the eager call"
    del graph
    torch.cuda.synchronize()
