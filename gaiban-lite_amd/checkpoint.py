"""Loader of DeepSeek-V4-Flash MoE layers from a safetensors checkpoint.

Restates the reference's load path for the layer's MoE half
(``runtime/dsv4_direct/checkpoint.py:403-428`` ``load_weight_map``,
``runtime/dsv4_direct/ops/marlin_moe.py:225-401`` ``ShardReader`` and
``load_resident_moe_layer``, ``runtime/dsv4_direct/block_weights.py:135-150,
805-815`` for the gate): tensors are located only through
``model.safetensors.index.json``'s ``weight_map``, read with safetensors
slices (a tensor-parallel rank reads only its intermediate-dimension slice),
and become resident in this library's formats:

* routed experts ``{prefix}.experts.{e}.w1|w3|w2.weight`` (MXFP4 E2M1 codes,
  two per byte, stored as I8) and ``.scale`` (E8M0, one per 32 K) ->
  ``ResidentMXFP4MoEWeights`` (w1 and w3 stacked as W13 = [w1; w3], the
  reference's concatenation order, then the device byte permutation into MFMA
  tiles; the values are not requantised);
* the shared expert ``{prefix}.shared_experts.w1|w3|w2.weight`` (FP8 E4M3)
  with ``.scale`` (E8M0 per 128 x 128 block) -> ``ResidentFP8SharedExpert``;
* the gate ``{prefix}.gate.weight`` (bf16 [E, H]) with ``.bias`` (fp32 [E],
  learned routing) or ``.tid2eid`` (int64 [vocab, k], hash routing) ->
  ``ResidentGateWeights``.

Checkpoint tensors are read with safetensors (no pickle).  The file set is
whatever the index names; shards are opened once each and closed on exit.
"""

from __future__ import annotations

import hashlib
import json
import time
from pathlib import Path
from typing import Any, Callable

import torch

from .weights import ResidentFP8SharedExpert, ResidentMXFP4MoEWeights

INDEX_NAME = "model.safetensors.index.json"


class CheckpointContractError(ValueError):
    """The checkpoint's index or tensors do not match the expected layout."""


def load_weight_map(stage_root: Path) -> tuple[dict[str, str], dict[str, Any]]:
    """``model.safetensors.index.json`` -> (weight_map, meta) (``checkpoint.py:403-428``)."""

    index_path = Path(stage_root) / INDEX_NAME
    raw = index_path.read_bytes()
    document = json.loads(raw)
    weight_map = document.get("weight_map") if isinstance(document, dict) else None
    if not isinstance(weight_map, dict) or not weight_map:
        raise CheckpointContractError(f"{index_path}: missing or empty weight_map")
    for key, value in weight_map.items():
        if not isinstance(key, str) or not isinstance(value, str):
            raise CheckpointContractError(f"{index_path}: malformed weight_map entry {key!r}: {value!r}")
    return dict(weight_map), {
        "path": str(index_path),
        "index_sha256": hashlib.sha256(raw).hexdigest(),
        "weight_map_keys": len(weight_map),
    }


class ShardReader:
    """Tensors of a checkpoint, found only through the index ``weight_map``
    (the Flash runtime's sole shard-resolution rule, ``marlin_moe.py:225-262``).

    Each shard file is opened at most once, on first use, and stays open
    until ``close()`` (or the end of a ``with`` block).  A key the index does
    not list raises KeyError; a listed file outside the checkpoint directory
    raises CheckpointContractError."""

    def __init__(self, stage_root: Path, weight_map: dict[str, str]):
        self._root = Path(stage_root).resolve()
        self._file_of = dict(weight_map)
        self._open_files: dict[str, Any] = {}

    def _shard(self, key: str) -> Any:
        name = self._file_of.get(key)
        if name is None:
            raise KeyError(f"{key!r} is not listed in the index weight_map")
        shard = self._open_files.get(name)
        if shard is None:
            path = (self._root / name).resolve()
            if self._root not in path.parents:
                raise CheckpointContractError(f"weight_map names a file outside the checkpoint: {name}")
            from safetensors import safe_open

            shard = self._open_files[name] = safe_open(str(path), framework="pt", device="cpu")
        return shard

    def get_slice(self, key: str) -> Any:
        return self._shard(key).get_slice(key)

    def get_tensor(self, key: str) -> torch.Tensor:
        return self._shard(key).get_tensor(key)

    def read(self, key: str, index: Any = None) -> torch.Tensor:
        """The tensor, or its slice ``index``, as a contiguous CPU tensor."""

        t = self.get_tensor(key) if index is None else self.get_slice(key)[index]
        return t.contiguous()

    def close(self) -> None:
        shards, self._open_files = list(self._open_files.values()), {}
        for shard in shards:
            closer = getattr(shard, "close", None)
            if callable(closer):
                closer()

    def __enter__(self) -> "ShardReader":
        return self

    def __exit__(self, *exc_info: Any) -> None:
        self.close()


def _expect(t: torch.Tensor, key: str, shape: tuple[int, ...], dtypes: tuple[torch.dtype, ...]) -> torch.Tensor:
    if tuple(t.shape) != shape or t.dtype not in dtypes:
        names = "/".join(str(d) for d in dtypes)
        raise CheckpointContractError(f"{key}: expected {names} {list(shape)}, got {t.dtype} {list(t.shape)}")
    return t


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def tp_slice(intermediate_size: int, rank: int, world_size: int) -> tuple[int, int]:
    """This rank's [start, end) of the intermediate dimension; the bounds must
    keep the FP8 128-row blocks whole (``marlin_moe.py:301-307``)."""

    if world_size < 1 or not 0 <= rank < world_size:
        raise ValueError("rank must be in [0, world_size)")
    if intermediate_size % world_size:
        raise ValueError("intermediate size must divide the TP world size")
    local = intermediate_size // world_size
    start, end = rank * local, (rank + 1) * local
    if start % 128 or end % 128:
        raise ValueError("TP slice must preserve FP8 block boundaries")
    return start, end


def load_resident_mxfp4_layer(
    *,
    stage_root: Path,
    layer_id: int,
    hidden_size: int,
    intermediate_size: int,
    n_experts: int,
    device: torch.device,
    rank: int = 0,
    world_size: int = 1,
    key_prefix: str | None = None,
    checkpoint_id: str | None = None,
    progress: Callable[[str], None] | None = None,
    progress_every: int = 32,
    marlin_input_dtype: torch.dtype | None = None,
) -> ResidentMXFP4MoEWeights:
    """Routed experts (MXFP4) and the FP8 shared expert of one layer, this
    rank's intermediate slice (``load_resident_moe_layer``,
    ``marlin_moe.py:270-401``).  ``key_prefix`` overrides
    ``layers.{layer_id}.ffn`` (the MTP block uses ``mtp.0.ffn``);
    ``marlin_input_dtype=torch.float8_e4m3fn`` packs the routed experts for
    the W4A8 kernels."""

    start, end = tp_slice(intermediate_size, rank, world_size)
    local = end - start
    h = hidden_size
    prefix = key_prefix or f"layers.{layer_id}.ffn"
    weight_map, _ = load_weight_map(Path(stage_root))
    device = torch.device(device)
    started = time.perf_counter()
    w13 = torch.empty((n_experts, 2 * local, h // 2), dtype=torch.uint8, device=device)
    s13 = torch.empty((n_experts, 2 * local, h // 32), dtype=torch.uint8, device=device)
    w2 = torch.empty((n_experts, h, local // 2), dtype=torch.uint8, device=device)
    s2 = torch.empty((n_experts, h, local // 32), dtype=torch.uint8, device=device)
    codes = (torch.int8, torch.uint8)
    e8m0 = (torch.float8_e8m0fnu, torch.uint8)
    with ShardReader(Path(stage_root), weight_map) as reader:
        for e in range(n_experts):
            ex = f"{prefix}.experts.{e}"
            rows = slice(start, end)
            for j, name in enumerate(("w1", "w3")):
                wk, sk = f"{ex}.{name}.weight", f"{ex}.{name}.scale"
                w = _expect(reader.read(wk, rows), wk, (local, h // 2), codes)
                s = _expect(reader.read(sk, rows), sk, (local, h // 32), e8m0)
                w13[e, j * local:(j + 1) * local].copy_(_bytes(w), non_blocking=False)
                s13[e, j * local:(j + 1) * local].copy_(_bytes(s), non_blocking=False)
            wk, sk = f"{ex}.w2.weight", f"{ex}.w2.scale"
            w = _expect(reader.read(wk, (slice(None), slice(start // 2, end // 2))), wk, (h, local // 2), codes)
            s = _expect(reader.read(sk, (slice(None), slice(start // 32, end // 32))), sk, (h, local // 32), e8m0)
            w2[e].copy_(_bytes(w))
            s2[e].copy_(_bytes(s))
            if progress and progress_every and (e + 1) % progress_every == 0:
                progress(f"layer={layer_id} rank={rank} experts={e + 1}/{n_experts}")
        shared = load_shared_fp8(reader, prefix, h, start, end, device)
    resident = ResidentMXFP4MoEWeights.from_checkpoint_layout(
        w13, s13, w2, s2, experts=n_experts, has_shared=False, layer_id=layer_id, checkpoint_id=checkpoint_id,
        shared_fp8=shared, marlin_input_dtype=marlin_input_dtype,
    )
    del w13, s13, w2, s2
    torch.cuda.synchronize(device)
    resident.load_seconds = time.perf_counter() - started
    resident.rank, resident.world_size = rank, world_size
    resident.intermediate_start, resident.intermediate_end = start, end
    return resident


def _require_checkpoint_sha256(checkpoint_id) -> str:
    if (not isinstance(checkpoint_id, str) or len(checkpoint_id) != 64
            or any(c not in "0123456789abcdef" for c in checkpoint_id)):
        raise ValueError("resident MoE loads require a lowercase SHA-256 checkpoint_id (64 hex digits)")
    return checkpoint_id


def load_resident_moe_layer(
    *,
    stage_root: Path,
    layer_id: int,
    rank: int,
    world_size: int,
    hidden_size: int,
    intermediate_size: int,
    n_experts: int,
    device: torch.device,
    progress_every: int = 32,
    progress: Callable[[str], None] | None = None,
    checkpoint_id: str | None = None,
    key_prefix: str | None = None,
    marlin_input_dtype: torch.dtype | None = None,
) -> ResidentMXFP4MoEWeights:
    """The reference's loader entry under its own name and keywords
    (``runtime/dsv4_direct/ops/marlin_moe.py:270-300``): every routed expert of
    one layer (MXFP4) and the FP8 shared expert, this rank's intermediate
    slice, as resident tiles for this library's kernels.  ``checkpoint_id``
    must be the checkpoint's lowercase SHA-256 (ValueError otherwise, before
    anything is read); ``marlin_input_dtype`` None gives the W4A16 kernels'
    packing, ``torch.float8_e4m3fn`` the W4A8 kernels'.  The result carries
    ``layer_id``, ``rank``, ``world_size``, ``intermediate_start``,
    ``intermediate_end``, ``checkpoint_id``, ``marlin_input_dtype`` and
    ``load_seconds`` as the reference's resident record does."""

    _require_checkpoint_sha256(checkpoint_id)
    if marlin_input_dtype not in (None, torch.float8_e4m3fn):
        raise ValueError(f"marlin_input_dtype must be None or torch.float8_e4m3fn, not {marlin_input_dtype!r}")
    return load_resident_mxfp4_layer(
        stage_root=stage_root, layer_id=layer_id, hidden_size=hidden_size, intermediate_size=intermediate_size,
        n_experts=n_experts, device=device, rank=rank, world_size=world_size, key_prefix=key_prefix,
        checkpoint_id=checkpoint_id, progress=progress, progress_every=progress_every,
        marlin_input_dtype=marlin_input_dtype)


def load_shared_fp8(reader: ShardReader, prefix: str, hidden_size: int, start: int, end: int,
                    device: torch.device) -> ResidentFP8SharedExpert:
    """The FP8 shared expert's [start, end) intermediate slice (``marlin_moe.py:362-386``)."""

    sp = f"{prefix}.shared_experts"
    h, local = hidden_size, end - start
    rows, srows = slice(start, end), slice(start // 128, end // 128)
    fp8 = (torch.float8_e4m3fn, torch.uint8)
    e8m0 = (torch.float8_e8m0fnu, torch.uint8)
    parts = {}
    for name in ("w1", "w3"):
        wk, sk = f"{sp}.{name}.weight", f"{sp}.{name}.scale"
        parts[name] = _expect(reader.read(wk, rows), wk, (local, h), fp8)
        parts["s" + name[1]] = _expect(reader.read(sk, srows), sk, (local // 128, h // 128), e8m0)
    wk, sk = f"{sp}.w2.weight", f"{sp}.w2.scale"
    parts["w2"] = _expect(reader.read(wk, (slice(None), rows)), wk, (h, local), fp8)
    parts["s2"] = _expect(reader.read(sk, (slice(None), srows)), sk, (h // 128, local // 128), e8m0)
    dev = {k: _bytes(v).to(device) for k, v in parts.items()}
    return ResidentFP8SharedExpert.from_checkpoint(dev["w1"], dev["s1"], dev["w3"], dev["s3"], dev["w2"], dev["s2"])


def load_gate(*, stage_root: Path, layer_id: int, experts: int, hidden_size: int, device: torch.device,
              key_prefix: str | None = None, checkpoint_id: str | None = None):
    """``{prefix}.gate.weight`` with exactly one of ``.bias`` (learned) or
    ``.tid2eid`` (hash) (``block_weights.py:135-150,805-815``)."""

    from .moe_runtime import ResidentGateWeights

    prefix = key_prefix or f"layers.{layer_id}.ffn"
    weight_map, _ = load_weight_map(Path(stage_root))
    bias_key, hash_key = f"{prefix}.gate.bias", f"{prefix}.gate.tid2eid"
    if (bias_key in weight_map) == (hash_key in weight_map):
        raise CheckpointContractError(f"{prefix}.gate requires exactly one of bias or tid2eid")
    with ShardReader(Path(stage_root), weight_map) as reader:
        wk = f"{prefix}.gate.weight"
        weight = _expect(reader.read(wk), wk, (experts, hidden_size), (torch.bfloat16,)).to(device)
        bias = tid2eid = None
        if bias_key in weight_map:
            bias = _expect(reader.read(bias_key), bias_key, (experts,), (torch.float32,)).to(device)
        else:
            t = reader.read(hash_key)
            if t.ndim != 2 or t.dtype != torch.int64:
                raise CheckpointContractError(f"{hash_key}: expected int64 [vocab, k], got {t.dtype} {list(t.shape)}")
            tid2eid = t.to(device)
    return ResidentGateWeights(weight=weight, bias=bias, tid2eid=tid2eid, layer_id=layer_id,
                               checkpoint_id=checkpoint_id)


__all__ = [
    "CheckpointContractError",
    "INDEX_NAME",
    "ShardReader",
    "load_gate",
    "load_resident_moe_layer",
    "load_resident_mxfp4_layer",
    "load_shared_fp8",
    "load_weight_map",
    "tp_slice",
]
