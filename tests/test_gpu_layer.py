"""The ``TP4MoE`` drop-in on one GPU: gate GEMM, routing, the fused and the
staged launch chains, route overrides, alignment providers, hash routing, the
slot lifecycle and buffer sharing, checked against the CPU oracle.

Reference behaviour followed: ``moe_runtime.py:1565-1947`` (call path, slot
states, stage markers), ``:418-476`` (override validation), ``:631-666,
1812-1828`` (provider protocol), ``moe_forward.py:186-231`` (hash gate).
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    MoERouteOverride,
    ResidentGateWeights,
    ResidentInt4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    synthetic as S,
)
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size
from helpers import DeviceExpertSource, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SHAPE = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
SCORES = {"sigmoid": O.SCORE_SIGMOID, "softmax": O.SCORE_SOFTMAX, "sqrtsoftplus": O.SCORE_SQRTSOFTPLUS}
_CACHE: dict = {}


def resident():
    if "res" not in _CACHE:
        w13, s13, w2, s2 = S.make_checkpoint_experts(SHAPE, seed=7, device=DEV)
        _CACHE["res"] = ResidentInt4MoEWeights.from_checkpoint_layout(
            w13, s13, w2, s2, experts=SHAPE.experts, has_shared=True)
        _CACHE["src"] = DeviceExpertSource(w13, s13, w2, s2)
    return _CACHE["res"], _CACHE["src"]


def make_layer(*, score="sqrtsoftplus", route_scale=1.5, clamp=10.0, bias=True, rows=(64,),
               slots=1, provider=None, tid2eid=None, donor=None):
    res, _ = resident()
    g = torch.Generator(DEV).manual_seed(11)
    wg = (torch.randn((SHAPE.experts, SHAPE.hidden), device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    b = None
    if bias and tid2eid is None:
        b = torch.randn((SHAPE.experts,), device=DEV, generator=g) * 0.05
    gate = ResidentGateWeights(weight=wg, bias=b, tid2eid=tid2eid)
    cfg = TP4MoEConfig(hidden_size=SHAPE.hidden, intermediate_size=SHAPE.inter,
                       experts=SHAPE.experts, topk=SHAPE.topk, route_scale=route_scale,
                       clamp_limit=clamp, score_func=score, shared_experts=1)
    return TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=rows,
                  slots_per_shape=slots, alignment_provider=provider, buffer_donor=donor)


def hidden(rows, seed=1):
    return S.make_hidden(rows, SHAPE.hidden, seed=seed, device=DEV).view(1, rows, SHAPE.hidden)


def oracle_out(layer, x, ids, weights):
    _, src = resident()
    return O.moe_fp32(to_np_f32(x.view(-1, SHAPE.hidden)), np.asarray(ids), np.asarray(weights), src,
                      shared_index=SHAPE.experts, clamp_limit=layer.config.clamp_limit)


@pytest.mark.parametrize("score", list(SCORES))
def test_gate_gemm_routing_and_output(score):
    print(f"[layer] gate GEMM + {score}", flush=True)
    layer = make_layer(score=score)
    x = hidden(64)
    with layer.observe_route_tensors(capture_local_input=True) as seen:
        out, trace = layer(x)
    torch.cuda.synchronize()
    r = seen[0]
    # gate GEMM: fp32 accumulation of bf16 x . Wg^T
    ref_logits = x.view(64, -1).float() @ layer.gate.weight.float().T
    torch.testing.assert_close(r.gate_logits, ref_logits, rtol=1e-4, atol=1e-4)
    logits = r.gate_logits.cpu().numpy()
    bias = layer.gate.bias.cpu().numpy()
    ref = O.route_topk(logits, SHAPE.topk, score_func=SCORES[score], bias=bias,
                       route_scale=layer.config.route_scale)
    np.testing.assert_array_equal(r.ids.cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(r.weights.cpu().numpy().view(np.uint32), ref.weights.view(np.uint32))
    np.testing.assert_array_equal(r.margin.cpu().numpy().view(np.uint32), ref.margin.view(np.uint32))
    assert trace.route_ids_row_zero == tuple(int(v) for v in ref.ids[0])
    assert torch.equal(r.local_input, x.view(64, -1))
    assert_moe_close(to_np_f32(out.view(64, -1)), oracle_out(layer, x, ref.ids, ref.weights),
                     what=f"layer {score}")


def test_fused_and_staged_chains_are_bit_identical():
    layer = make_layer()
    x = hidden(64, seed=3)
    fused, _ = layer(x)
    marks = []
    staged, _ = layer(x, stage_marker=marks.append)
    torch.cuda.synchronize()
    assert torch.equal(fused, staged)
    assert marks == [
        "moe_inputs_ready", "moe_hidden_all_gather_done", "moe_ids_all_gather_done",
        "moe_route_done", "moe_routed_done", "moe_shared_done", "moe_combine_done",
        "moe_reduce_scatter_done", "moe_finalize_done",
    ]
    # forward_tensor is the same computation without a trace
    ft = layer.forward_tensor(x)
    torch.cuda.synchronize()
    assert torch.equal(ft, fused)


def test_router_logits_argument_skips_gate_gemm():
    layer = make_layer(score="sigmoid", route_scale=1.0, clamp=0.0, bias=False)
    x = hidden(64, seed=4)
    logits = S.make_logits(64, SHAPE.experts, seed=5, device=DEV)
    out, trace = layer(x, router_logits=logits)
    torch.cuda.synchronize()
    ref = O.route_topk(logits.cpu().numpy(), SHAPE.topk, score_func=O.SCORE_SIGMOID)
    assert trace.route_ids_row_zero == tuple(int(v) for v in ref.ids[0])
    assert_moe_close(to_np_f32(out.view(64, -1)), oracle_out(layer, x, ref.ids, ref.weights),
                     what="router_logits")


def test_route_override():
    layer = make_layer()
    x = hidden(64, seed=6)
    g = torch.Generator(DEV).manual_seed(9)
    ids = torch.stack([torch.randperm(SHAPE.experts, device=DEV, generator=g)[:SHAPE.topk]
                       for _ in range(64)]).to(torch.int32)
    w = torch.rand((64, SHAPE.topk), device=DEV, generator=g) + 0.1
    w = (w / w.sum(dim=1, keepdim=True) * layer.config.route_scale).float()
    out, trace = layer(x, route_override=MoERouteOverride(ids=ids, weights=w))
    torch.cuda.synchronize()
    assert trace.route_source == "explicit_global"
    assert trace.route_ids_row_zero == tuple(int(v) for v in ids[0].cpu())
    assert_moe_close(to_np_f32(out.view(64, -1)), oracle_out(layer, x, ids.cpu(), w.cpu()),
                     what="override")
    # duplicate ids in a row are a contract violation, raised before any launch
    bad = ids.clone()
    bad[0, 1] = bad[0, 0]
    with pytest.raises(ValueError):
        layer(x, route_override=MoERouteOverride(ids=bad, weights=w))
    assert layer.slot_completion_status(64, 0)["state"] == "free"


class _Provider:
    """Alignment provider owning its storage, filling the caller's output."""

    def __init__(self, wrong_output=False):
        self.scratch = torch.zeros(16, dtype=torch.int32, device=DEV)
        self.calls = 0
        self.wrong_output = wrong_output

    def storage_tensors(self):
        return (self.scratch,)

    def __call__(self, route_ids, *, block_size, num_experts, output, slot):
        self.calls += 1
        got = deterministic_moe_align_block_size(route_ids, block_size=block_size,
                                                 num_experts=num_experts, output=output)
        if self.wrong_output:
            return deterministic_moe_align_block_size(route_ids, block_size=block_size,
                                                      num_experts=num_experts)
        return got


def test_alignment_provider_protocol():
    base = make_layer()
    x = hidden(64, seed=8)
    ref, _ = base(x)
    prov = _Provider()
    layer = make_layer(provider=prov)
    out, _ = layer(x)
    torch.cuda.synchronize()
    assert prov.calls == 1
    assert torch.equal(out, ref)

    bad = make_layer(provider=_Provider(wrong_output=True))
    with pytest.raises(RuntimeError):
        bad(x)
    # the lifecycle is poisoned: every slot refuses further calls
    with pytest.raises(RuntimeError):
        bad(x)
    assert bad.slot_completion_status(64, 0)["state"] == "poisoned"


def test_hash_gate():
    vocab = 97
    g = torch.Generator(DEV).manual_seed(13)
    tid2eid = torch.stack([torch.randperm(SHAPE.experts, device=DEV, generator=g)[:SHAPE.topk]
                           for _ in range(vocab)]).to(torch.int64)
    layer = make_layer(tid2eid=tid2eid, rows=(48,))
    x = hidden(48, seed=10)
    input_ids = torch.randint(0, vocab, (1, 48), device=DEV, generator=g, dtype=torch.int64)
    with layer.observe_route_tensors() as seen:
        out, trace = layer(x, input_ids_local=input_ids)
    torch.cuda.synchronize()
    logits = seen[0].gate_logits.cpu().numpy()
    ref = O.hash_route(logits, tid2eid.cpu().numpy(), input_ids.view(-1).cpu().numpy(),
                       route_scale=layer.config.route_scale)
    np.testing.assert_array_equal(seen[0].ids.cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(seen[0].weights.cpu().numpy().view(np.uint32), ref.weights.view(np.uint32))
    assert_moe_close(to_np_f32(out.view(48, -1)), oracle_out(layer, x, ref.ids, ref.weights), what="hash")
    with pytest.raises(ValueError):
        layer(x)  # hash routing needs input ids
    # a token id outside the table: by default no host read, the output is NaN
    bad_ids = input_ids.clone()
    bad_ids[0, 5] = vocab
    poisoned, _ = layer(x, input_ids_local=bad_ids)
    torch.cuda.synchronize()
    assert torch.isnan(poisoned.float()).all()
    # opted in, the eager call is refused before any launch
    layer.check_hash_token_ids = True
    with pytest.raises(ValueError, match="outside"):
        layer(x, input_ids_local=bad_ids)
    layer.check_hash_token_ids = False
    again, _ = layer(x, input_ids_local=input_ids)
    torch.cuda.synchronize()
    assert torch.equal(again, out)


def test_slots_shapes_and_buffer_donor():
    layer = make_layer(rows=(1, 64), slots=2)
    assert layer.registered_global_rows == (1, 64)
    assert layer.registered_slots == {1: (0, 1), 64: (0, 1)}
    x = hidden(64, seed=12)
    a, _ = layer(x, slot=0)
    b, _ = layer(x, slot=1)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert a.data_ptr() != b.data_ptr()  # owning clones
    one, _ = layer(hidden(1, seed=14))
    torch.cuda.synchronize()
    assert one.shape == (1, 1, SHAPE.hidden)
    with pytest.raises(ValueError):
        layer(hidden(32))  # unregistered row count
    st = layer.slot_completion_status(64, 1)
    assert st == {"state": "free", "has_completion_event": True}
    layer.reset_free_slot_completion_event(64, 1)
    assert layer.slot_completion_status(64, 1)["has_completion_event"] is False

    other = make_layer(rows=(64,), donor=layer)
    c, _ = other(x, slot=1)
    torch.cuda.synchronize()
    assert torch.equal(c, a)
