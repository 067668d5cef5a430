"""CPU checks of the checkpoint loader's host side: the index weight_map is
the only shard resolution (``checkpoint.py:403-428``), slices come back with
the checkpoint's dtypes, keys outside the index or files outside the
checkpoint are refused, TP slices keep 128-row blocks whole, and the gate
loads with exactly one of bias / tid2eid."""

import json

import pytest
import torch

from checkpoint_fixture import write_checkpoint
from gaiban_lite_amd import checkpoint as C


def test_weight_map_and_slices(tmp_path):
    raw = write_checkpoint(tmp_path, layer_id=3, experts=4, hidden=512, inter=512)
    wm, meta = C.load_weight_map(tmp_path)
    assert set(wm) == set(raw) and meta["weight_map_keys"] == len(raw) and len(meta["index_sha256"]) == 64
    assert len(set(wm.values())) == 2
    with C.ShardReader(tmp_path, wm) as r:
        key = "layers.3.ffn.experts.2.w2.weight"
        sl = r.read(key, (slice(None), slice(64, 128)))
        assert sl.dtype == torch.int8 and torch.equal(sl, raw[key][:, 64:128])
        s = r.read("layers.3.ffn.shared_experts.w1.scale")
        assert s.dtype == torch.float8_e8m0fnu and torch.equal(s.view(torch.uint8),
                                                               raw["layers.3.ffn.shared_experts.w1.scale"].view(torch.uint8))
        with pytest.raises(KeyError, match="not listed in the index"):
            r.read("layers.3.ffn.experts.9.w1.weight")


def test_index_validation(tmp_path):
    (tmp_path / C.INDEX_NAME).write_text(json.dumps({"weight_map": {}}))
    with pytest.raises(C.CheckpointContractError, match="weight_map"):
        C.load_weight_map(tmp_path)
    (tmp_path / C.INDEX_NAME).write_text(json.dumps({"weight_map": {"a": "../outside.safetensors"}}))
    wm, _ = C.load_weight_map(tmp_path)
    with C.ShardReader(tmp_path, wm) as r, pytest.raises(C.CheckpointContractError, match="outside"):
        r.read("a")


def test_tp_slice_rules():
    assert C.tp_slice(2048, 0, 4) == (0, 512) and C.tp_slice(2048, 3, 4) == (1536, 2048)
    with pytest.raises(ValueError, match="block"):
        C.tp_slice(2048, 1, 32)   # 64-row slices split the 128-row scale blocks
    with pytest.raises(ValueError):
        C.tp_slice(2048, 4, 4)


@pytest.mark.parametrize("hash_gate", [False, True])
def test_gate_loads_learned_or_hash(tmp_path, hash_gate):
    raw = write_checkpoint(tmp_path, layer_id=0, experts=8, hidden=512, inter=512, hash_gate=hash_gate)
    gate = C.load_gate(stage_root=tmp_path, layer_id=0, experts=8, hidden_size=512, device="cpu")
    assert torch.equal(gate.weight, raw["layers.0.ffn.gate.weight"])
    if hash_gate:
        assert gate.route_kind == "hash" and gate.bias is None
        assert torch.equal(gate.tid2eid, raw["layers.0.ffn.gate.tid2eid"])
    else:
        assert gate.route_kind == "learned" and torch.equal(gate.bias, raw["layers.0.ffn.gate.bias"])
    with pytest.raises(C.CheckpointContractError, match="expected"):
        C.load_gate(stage_root=tmp_path, layer_id=0, experts=16, hidden_size=512, device="cpu")
