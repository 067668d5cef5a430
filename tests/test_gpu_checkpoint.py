"""Loading a layer from a safetensors checkpoint (index + shards with the
Flash checkpoint's names and dtypes) into the MXFP4 routed experts and the
FP8 shared expert: the resident tensors equal those built from the same raw
tensors in memory (world size 1, and rank 1 of 2 against the sliced
tensors), and the loaded layer's output matches the oracle on the raw
checkpoint values to max_rel and rel_fro <= 1e-2."""

import numpy as np
import pytest
import torch

import oracle as O
from checkpoint_fixture import write_checkpoint
from gaiban_lite_amd import (
    ResidentFP8SharedExpert,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    checkpoint as C,
    synthetic as S,
)
from helpers import assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
E, H, I = 8, 512, 1024


def stacked(raw, p, e_range, lo, hi):
    w13 = torch.stack([torch.cat([raw[f"{p}.experts.{e}.w1.weight"][lo:hi], raw[f"{p}.experts.{e}.w3.weight"][lo:hi]])
                       for e in e_range]).view(torch.uint8)
    s13 = torch.stack([torch.cat([raw[f"{p}.experts.{e}.w1.scale"][lo:hi], raw[f"{p}.experts.{e}.w3.scale"][lo:hi]])
                       for e in e_range]).view(torch.uint8)
    w2 = torch.stack([raw[f"{p}.experts.{e}.w2.weight"][:, lo // 2:hi // 2] for e in e_range]).view(torch.uint8)
    s2 = torch.stack([raw[f"{p}.experts.{e}.w2.scale"][:, lo // 32:hi // 32] for e in e_range]).view(torch.uint8)
    return [t.contiguous().to(DEV) for t in (w13, s13, w2, s2)]


def shared_raw(raw, p, lo, hi):
    sp = f"{p}.shared_experts"
    b = lambda k, ix: raw[k][ix].contiguous().view(torch.uint8).to(DEV)
    rows, srows = slice(lo, hi), slice(lo // 128, hi // 128)
    return (b(f"{sp}.w1.weight", rows), b(f"{sp}.w1.scale", srows), b(f"{sp}.w3.weight", rows),
            b(f"{sp}.w3.scale", srows), b(f"{sp}.w2.weight", (slice(None), rows)),
            b(f"{sp}.w2.scale", (slice(None), srows)))


@pytest.mark.parametrize("rank,world", [(0, 1), (1, 2)])
def test_loaded_residents_equal_in_memory_build(tmp_path, rank, world):
    print(f"[checkpoint] rank {rank} of {world}", flush=True)
    raw = write_checkpoint(tmp_path, layer_id=5, experts=E, hidden=H, inter=I)
    res = C.load_resident_mxfp4_layer(stage_root=tmp_path, layer_id=5, hidden_size=H, intermediate_size=I,
                                      n_experts=E, device=DEV, rank=rank, world_size=world)
    lo, hi = C.tp_slice(I, rank, world)
    want = ResidentMXFP4MoEWeights.from_checkpoint_layout(
        *stacked(raw, "layers.5.ffn", range(E), lo, hi), experts=E, has_shared=False,
        shared_fp8=ResidentFP8SharedExpert.from_checkpoint(*shared_raw(raw, "layers.5.ffn", lo, hi)))
    torch.cuda.synchronize()
    for name in ("w13_q", "w13_s", "w2_q", "w2_s"):
        assert torch.equal(getattr(res, name), getattr(want, name)), name
    for name in ("w13_q", "w13_s", "w2_q", "w2_s"):
        assert torch.equal(getattr(res.shared_fp8, name), getattr(want.shared_fp8, name)), "shared " + name
    assert res.layer_id == 5 and res.load_seconds is not None and res.intermediate_size == hi - lo


def test_loaded_layer_matches_oracle(tmp_path):
    print("[checkpoint] layer forward", flush=True)
    raw = write_checkpoint(tmp_path, layer_id=7, experts=E, hidden=H, inter=I, seed=4)
    res = C.load_resident_mxfp4_layer(stage_root=tmp_path, layer_id=7, hidden_size=H, intermediate_size=I,
                                      n_experts=E, device=DEV)
    gate = C.load_gate(stage_root=tmp_path, layer_id=7, experts=E, hidden_size=H, device=DEV)
    cfg = TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=2, route_scale=1.5, clamp_limit=10.0,
                       score_func="sqrtsoftplus", shared_experts=1)
    layer = TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[64])
    x = S.make_hidden(64, H, seed=3, device=DEV)
    lg = S.make_logits(64, E, seed=4, device=DEV)
    out = layer.forward_tensor(x.view(1, 64, H), router_logits=lg)
    torch.cuda.synchronize()
    p = "layers.7.ffn"
    r = O.route_topk(lg.cpu().numpy(), 2, score_func=O.SCORE_SQRTSOFTPLUS,
                     bias=raw[f"{p}.gate.bias"].numpy(), route_scale=1.5)
    w13, s13, w2, s2 = [t.cpu().numpy() for t in stacked(raw, p, range(E), 0, I)]
    src = O.MXFP4ExpertSource(w13, s13, w2, s2)
    xf = to_np_f32(x)
    routed = O.bf16_round(O.moe_fp32(xf, r.ids, r.weights, src, shared_index=None, clamp_limit=10.0))
    sh = [t.cpu().numpy() for t in shared_raw(raw, p, 0, I)]
    want = O.bf16_round(routed + O.shared_fp8_bf16(xf, *sh, 10.0))
    assert_moe_close(to_np_f32(out.view(64, H)), want, what="checkpoint layer")


def test_loaded_hash_layer_matches_oracle(tmp_path):
    """A hash-routed layer (the checkpoint's layers 0-2: gate.tid2eid, no
    bias) loaded from the safetensors files: token ids pick the experts,
    sqrt-softplus scores of the gate logits weight them (``moe_forward.py:
    186-231``); MXFP4 routed experts plus the FP8 shared expert."""

    print("[checkpoint] hash layer forward", flush=True)
    vocab = 50
    raw = write_checkpoint(tmp_path, layer_id=1, experts=E, hidden=H, inter=I, seed=6, hash_gate=True, vocab=vocab,
                           topk=2)
    res = C.load_resident_mxfp4_layer(stage_root=tmp_path, layer_id=1, hidden_size=H, intermediate_size=I,
                                      n_experts=E, device=DEV)
    gate = C.load_gate(stage_root=tmp_path, layer_id=1, experts=E, hidden_size=H, device=DEV)
    assert gate.route_kind == "hash"
    cfg = TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=2, route_scale=1.5, clamp_limit=10.0,
                       score_func="sqrtsoftplus", shared_experts=1)
    layer = TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[48])
    x = S.make_hidden(48, H, seed=8, device=DEV).view(1, 48, H)
    input_ids = torch.randint(0, vocab, (1, 48), device=DEV, generator=torch.Generator(DEV).manual_seed(3),
                              dtype=torch.int64)
    with layer.observe_route_tensors() as seen:
        out, _ = layer(x, input_ids_local=input_ids)
    torch.cuda.synchronize()
    p = "layers.1.ffn"
    ref = O.hash_route(seen[0].gate_logits.cpu().numpy(), raw[f"{p}.gate.tid2eid"].numpy(),
                       input_ids.view(-1).cpu().numpy(), route_scale=1.5)
    np.testing.assert_array_equal(seen[0].ids.cpu().numpy(), ref.ids)
    w13, s13, w2, s2 = [t.cpu().numpy() for t in stacked(raw, p, range(E), 0, I)]
    xf = to_np_f32(x.view(48, H))
    routed = O.bf16_round(O.moe_fp32(xf, ref.ids, ref.weights, O.MXFP4ExpertSource(w13, s13, w2, s2),
                                     shared_index=None, clamp_limit=10.0))
    sh = [t.cpu().numpy() for t in shared_raw(raw, p, 0, I)]
    want = O.bf16_round(routed + O.shared_fp8_bf16(xf, *sh, 10.0))
    assert_moe_close(to_np_f32(out.view(48, H)), want, what="checkpoint hash layer")
