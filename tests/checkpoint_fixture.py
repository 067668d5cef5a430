"""Writes a small synthetic DeepSeek-V4-Flash-style checkpoint (index +
safetensors shards, tensor names and dtypes of the Flash checkpoint contract,
``experiments/A0-flash-checkpoint-contract/flash-contract.txt``) for loader
tests.  Test infrastructure: the values come from the seeded synthetic
generators."""

import json
from pathlib import Path

import torch
from safetensors.torch import save_file

from gaiban_lite_amd import synthetic as S


def write_checkpoint(root: Path, *, layer_id: int, experts: int, hidden: int, inter: int, hash_gate: bool = False,
                     vocab: int = 64, topk: int = 2, seed: int = 0, shards: int = 2) -> dict:
    """Returns the raw CPU tensors by name."""

    shape = S.LayerShape(experts=experts, hidden=hidden, inter=inter, topk=topk, has_shared=False)
    w13, s13, w2, s2 = S.make_checkpoint_experts_mxfp4(shape, seed=seed, device="cpu")
    p = f"layers.{layer_id}.ffn"
    t = {}
    for e in range(experts):
        t[f"{p}.experts.{e}.w1.weight"] = w13[e, :inter].contiguous().view(torch.int8)
        t[f"{p}.experts.{e}.w3.weight"] = w13[e, inter:].contiguous().view(torch.int8)
        t[f"{p}.experts.{e}.w1.scale"] = s13[e, :inter].contiguous().view(torch.float8_e8m0fnu)
        t[f"{p}.experts.{e}.w3.scale"] = s13[e, inter:].contiguous().view(torch.float8_e8m0fnu)
        t[f"{p}.experts.{e}.w2.weight"] = w2[e].contiguous().view(torch.int8)
        t[f"{p}.experts.{e}.w2.scale"] = s2[e].contiguous().view(torch.float8_e8m0fnu)
    for name, (n, k), sd in (("w1", (inter, hidden), 1), ("w3", (inter, hidden), 2), ("w2", (hidden, inter), 3)):
        q, s = S.make_fp8_block_linear(n, k, seed=seed + sd, device="cpu", std=0.03)
        t[f"{p}.shared_experts.{name}.weight"] = q.view(torch.float8_e4m3fn)
        t[f"{p}.shared_experts.{name}.scale"] = s.view(torch.float8_e8m0fnu)
    g = torch.Generator().manual_seed(seed + 11)
    t[f"{p}.gate.weight"] = (torch.randn((experts, hidden), generator=g) * 0.03).to(torch.bfloat16)
    if hash_gate:
        t[f"{p}.gate.tid2eid"] = torch.stack([torch.randperm(experts, generator=g)[:topk] for _ in range(vocab)])
    else:
        t[f"{p}.gate.bias"] = torch.randn((experts,), generator=g) * 0.05
    t[f"layers.{layer_id}.ffn_norm.weight"] = torch.ones(hidden, dtype=torch.bfloat16)  # an unrelated key
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    names = sorted(t)
    weight_map = {}
    for i in range(shards):
        part = names[i::shards]
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: t[k] for k in part}, str(root / fname))
        weight_map.update({k: fname for k in part})
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return t
