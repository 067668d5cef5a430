"""Single-GPU MoE layer with the ``TP4MoE`` call signature.

Drop-in for ``runtime/dsv4_direct/moe_runtime.py:TP4MoE`` at world size 1: the
whole unsharded layer (all routed experts plus the shared expert) is resident
on one MI355X, so the all_gather / reduce_scatter of the reference
(``moe_runtime.py:1699,1893``) are identities and the stage markers around
them fire back to back.  The compute between them -- gate, alignment, grouped
experts, top-k combine, shared expert and add (``moe_runtime.py:1714-1888``)
-- runs in the HIP kernels behind ``include/dsv4moe.h``.

Kept from the reference: constructor keywords, per-(rows, slot) preallocated
buffers with the ``free -> in_flight -> free | poisoned`` lifecycle and a
per-slot completion event, route override validation
(``moe_runtime.py:418-476``), the alignment-provider protocol
(``:631-666,1812-1828``), stage markers, ``MoETrace``, ``forward_tensor``,
route observation and the slot-status introspection used by graph callers.
"""

from __future__ import annotations

import hashlib
import math
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any, Callable, Iterable, Iterator

import torch

from . import contracts as C
from . import ops
from .deterministic_moe_align import (
    DeterministicMoEAlignment,
    allocate_deterministic_moe_alignment,
)
from .weights import ResidentInt4MoEWeights, ResidentMXFP4MoEWeights

SCORE_FUNCS = ("sigmoid", "softmax", "sqrtsoftplus")


@dataclass(frozen=True)
class TP4MoEConfig:
    """Layer geometry and routing contract.

    The reference pins the Flash geometry and TP world 4
    (``moe_runtime.py:35-67``); this build runs the whole layer on one GPU
    (``world_size`` 1) and accepts any geometry the kernels support.
    ``FLASH_CONFIG`` is the DeepSeek-V4-Flash contract.
    """

    hidden_size: int = 4096
    intermediate_size: int = 2048
    experts: int = 256
    topk: int = 6
    route_scale: float = 1.5
    clamp_limit: float = 10.0
    world_size: int = 1
    score_func: str = "sqrtsoftplus"
    shared_experts: int = 1

    @property
    def local_intermediate(self) -> int:
        return self.intermediate_size // self.world_size

    def validate(self) -> None:
        if self.world_size != 1:
            raise ValueError(
                "this build keeps the whole MoE layer on one GPU: world_size must be 1"
            )
        for name in ("hidden_size", "intermediate_size"):
            value = getattr(self, name)
            if not isinstance(value, int) or value <= 0 or value % 256:
                raise ValueError(f"{name} must be a positive multiple of 256")
        if not isinstance(self.experts, int) or not 1 <= self.experts <= 1024:
            raise ValueError("experts must be in [1, 1024]")
        if not isinstance(self.topk, int) or not 1 <= self.topk < self.experts or self.topk > 16:
            raise ValueError("topk must be in [1, min(experts - 1, 16)]")
        if not math.isfinite(self.route_scale) or self.route_scale <= 0:
            raise ValueError("route_scale must be finite and positive")
        if not math.isfinite(self.clamp_limit) or self.clamp_limit < 0:
            raise ValueError("clamp_limit must be finite and >= 0 (0 disables the clamp)")
        if self.score_func not in SCORE_FUNCS:
            raise ValueError(f"score_func must be one of {SCORE_FUNCS}")
        if self.shared_experts not in (0, 1):
            raise ValueError("shared_experts must be 0 or 1")


FLASH_CONFIG = TP4MoEConfig()


@dataclass
class ResidentGateWeights:
    """Gate parameters (``runtime/dsv4_direct/block_weights.py:135-150``).

    ``weight`` bf16 [E, H]; ``bias`` fp32 [E] (selection shift) or None;
    ``tid2eid`` int64 [vocab, k] for hash layers.  A hash gate has no bias.
    """

    weight: torch.Tensor
    bias: torch.Tensor | None = None
    layer_id: int | None = None
    rank: int | None = None
    world_size: int | None = None
    checkpoint_id: str | None = None
    tid2eid: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.tid2eid is not None and self.bias is not None:
            raise ValueError("a hash gate (tid2eid) forbids a bias")

    @property
    def route_kind(self) -> str:
        return "hash" if self.tid2eid is not None else "learned"


@dataclass(frozen=True)
class MoETrace:
    local_input_shape: tuple[int, ...]
    gathered_shape: tuple[int, ...]
    partial_shape: tuple[int, ...]
    local_output_shape: tuple[int, ...]
    route_ids_row_zero: tuple[int, ...]
    route_weights_row_zero: tuple[float, ...]
    route_margin_min: float | None
    route_digest: str
    stage_digests: dict[str, str]
    buffer_slot: int
    shared_path: str = "int4_g128_fused_grouped"
    route_source: str = "native"


@dataclass(frozen=True)
class MoERouteOverride:
    """Explicit full route (ids int32 [rows, k], weights fp32 [rows, k])."""

    ids: torch.Tensor
    weights: torch.Tensor


@dataclass(frozen=True)
class MoERouteTensors:
    weights: torch.Tensor
    ids: torch.Tensor
    margin: torch.Tensor | None
    selection_ids: torch.Tensor | None
    selection_scores: torch.Tensor | None
    local_input: torch.Tensor | None = None
    gate_logits: torch.Tensor | None = None
    route_source: str = "native"


@dataclass
class _LayerBuffers:
    workspace: torch.Tensor
    logits: torch.Tensor
    route_ids: torch.Tensor
    route_weights: torch.Tensor
    margin: torch.Tensor
    alignment: DeterministicMoEAlignment
    block_size_m: int
    ready_event: Any
    gathered_input_ids: torch.Tensor | None = None
    shared_workspace: torch.Tensor | None = None  # FP8-block shared expert
    has_completion_event: bool = False
    state: str = "free"


def _tensor_digest(*tensors: torch.Tensor) -> str:
    digest = hashlib.sha256()
    for tensor in tensors:
        digest.update(f"{list(tensor.shape)}|{tensor.dtype}|".encode())
        digest.update(tensor.detach().contiguous().view(torch.uint8).cpu().numpy().tobytes())
    return digest.hexdigest()


def _snapshot_route_override(
    value: MoERouteOverride, *, rows: int, config: TP4MoEConfig, device: torch.device
) -> tuple[torch.Tensor, torch.Tensor]:
    """An owned, validated copy of an injected route (the contract of the
    reference's override path, ``moe_runtime.py:418-476``): ids int32 and
    weights fp32, both [rows, k] on the layer's device; ids unique per row
    and inside [0, experts); weights finite, positive, and for renormalised
    score functions summing to route_scale per row.  Reads the device."""

    if not isinstance(value, MoERouteOverride):
        raise TypeError(f"route_override: expected MoERouteOverride, got {type(value).__name__}")
    want = (rows, config.topk)
    ids = C.tensor("route_override.ids", value.ids, shape=want, dtype=torch.int32, device=device,
                   contiguous=True, no_grad=True).detach().clone()
    weights = C.tensor("route_override.weights", value.weights, shape=want, dtype=torch.float32, device=device,
                       contiguous=True, no_grad=True).detach().clone()
    C.route_weights("route_override.weights", weights,
                    row_sum=None if config.score_func == "softmax" else float(config.route_scale))
    C.expert_table("route_override.ids", ids, experts=config.experts)
    return ids, weights


@dataclass(frozen=True)
class MoERouteCaptureBuffer:
    """Stable device storage that a captured layer call writes its effective
    route into (``moe_runtime.py:121-136``): ids int32 [rows, k] (-1 until
    written), weights fp32 [rows, k], and a device generation counter that
    every call adds one to."""

    global_rows: int
    slot: int
    owner_id: int
    ids: torch.Tensor
    weights: torch.Tensor
    generation: torch.Tensor
    tensor_pointers: tuple[int, int, int]

    @property
    def resident_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.ids, self.weights, self.generation))


@dataclass(frozen=True)
class MoERouteCaptureEvidence:
    """A host copy of one capture buffer taken outside replay
    (``moe_runtime.py:138-148``)."""

    global_rows: int
    slot: int
    ids: torch.Tensor
    weights: torch.Tensor
    generation: int
    device_tensor_pointers: tuple[int, int, int]
    route_digest: str


class TP4MoE:
    """Whole MoE layer resident on one GPU, ``TP4MoE``-compatible interface.

    Slots isolate storage, not ordering: calls are expected from one scheduler
    thread; every launch goes to the current stream of ``device``.
    """

    def __init__(
        self,
        *,
        config: TP4MoEConfig,
        resident: ResidentInt4MoEWeights | ResidentMXFP4MoEWeights,
        gate: ResidentGateWeights,
        rank: int = 0,
        device: torch.device,
        global_row_shapes: Iterable[int],
        group: Any = None,
        slots_per_shape: int = 1,
        alignment_provider: Callable[..., object] | None = None,
        marlin_input_dtype: torch.dtype | None = None,
        buffer_donor: "TP4MoE | None" = None,
    ) -> None:
        config.validate()
        device = torch.device(device)
        if device.type not in ("cuda", "cpu"):
            raise ValueError(f"TP4MoE runs on a GPU device, not {device}")
        # A layer built on the CPU supports the host-side lifecycle only
        # (registration, capture bindings, validation); every call raises.
        if rank != 0:
            raise ValueError("single-GPU layer: rank must be 0")
        if group is not None:
            import torch.distributed as dist

            if dist.is_initialized() and dist.get_world_size(group) != 1:
                raise ValueError("single-GPU layer: the process group must have world size 1")
        if marlin_input_dtype not in (None, torch.float8_e4m3fn):
            raise ValueError(f"unsupported input dtype {marlin_input_dtype!r}")
        if getattr(resident, "marlin_input_dtype", None) != marlin_input_dtype:
            raise ValueError(
                f"resident input dtype {getattr(resident, 'marlin_input_dtype', None)!r} "
                f"does not match requested {marlin_input_dtype!r}"
            )
        if marlin_input_dtype is not None and (config.hidden_size % 512 or config.intermediate_size % 512):
            raise ValueError("W4A8 needs hidden and intermediate sizes that are multiples of 512")
        if not isinstance(resident, (ResidentInt4MoEWeights, ResidentMXFP4MoEWeights)):
            raise TypeError("resident must be ResidentInt4MoEWeights or ResidentMXFP4MoEWeights")
        resident.validate()
        if (resident.experts, resident.hidden_size, resident.intermediate_size) != (
            config.experts, config.hidden_size, config.intermediate_size
        ):
            raise ValueError("resident expert geometry does not match the config")
        shared_fp8 = getattr(resident, "shared_fp8", None)
        if (resident.has_shared or shared_fp8 is not None) != bool(config.shared_experts):
            raise ValueError("resident shared-expert presence does not match the config")
        if resident.device != device:
            raise ValueError("resident weights must live on the configured device")
        if tuple(gate.weight.shape) != (config.experts, config.hidden_size):
            raise ValueError("gate weight shape mismatch")
        if gate.weight.device != device:
            raise ValueError("gate weight must use the configured device")
        if gate.bias is not None:
            if tuple(gate.bias.shape) != (config.experts,) or gate.bias.device != device:
                raise ValueError("gate bias must be [experts] on the configured device")
        if gate.tid2eid is not None:
            t = gate.tid2eid
            if t.ndim != 2 or t.shape[1] != config.topk or t.dtype != torch.int64 or t.device != device:
                raise ValueError(f"hash tid2eid must be int64 [vocab, {config.topk}] on the device")
            lo, hi = int(t.min().item()), int(t.max().item())
            if lo < 0 or hi >= config.experts:
                raise ValueError(f"hash route table range [{lo}, {hi}] outside [0, {config.experts})")
            ordered = t.sort(dim=1).values
            if bool((ordered[:, 1:] == ordered[:, :-1]).any().item()):
                raise ValueError("hash route table rows must contain unique expert IDs")
        if resident.checkpoint_id is not None and gate.checkpoint_id is not None:
            if resident.checkpoint_id != gate.checkpoint_id:
                raise ValueError("gate and MoE weights come from different checkpoints")

        self.config = config
        self.resident = resident
        self.gate = gate
        self.layer_id = resident.layer_id
        self.route_kind = gate.route_kind
        # Hash layers: when True, every eager call reads the token ids' range
        # back to the host and raises ValueError for an id outside the table
        # (a synchronisation per call).  When False (the default, as the
        # reference's forward), such an id makes the call's output NaN.
        self.check_hash_token_ids = False
        self.rank = 0
        self.device = device
        self.group = group
        self._marlin_input_dtype = marlin_input_dtype
        self._mxfp4 = isinstance(resident, ResidentMXFP4MoEWeights)
        # the W4A16 entries' scale ratios, computed once here (never inside a call,
        # which may be under graph capture); other formats take none
        self._ratio_kwargs: dict[str, torch.Tensor] = {}
        if not self._mxfp4 and marlin_input_dtype is None and device.type == "cuda":
            w13r, w2r = resident.scale_ratios()
            self._ratio_kwargs = {"w13r": w13r, "w2r": w2r}
        # shared expert: inside the grouped kernels (expert index E of the routed
        # stack) or, in the checkpoint FP8 format, as dense linears after them
        self._shared_fp8 = getattr(resident, "shared_fp8", None)
        self._grouped_shared = bool(config.shared_experts) and self._shared_fp8 is None
        self._gate_weight = gate.weight.to(torch.bfloat16).contiguous()
        self._gate_bias = None if gate.bias is None else gate.bias.float().contiguous()
        self.overlap_stats: dict[str, int] = {
            "overlapped_calls": 0,
            "overlapped_rows": 0,
            "sequential_calls": 0,
            "sequential_rows": 0,
        }
        self._route_tensor_observer: list[MoERouteTensors] | None = None
        self._route_observer_captures_local_input = False
        if alignment_provider is not None:
            if self.route_kind != "learned":
                raise ValueError("an injected alignment provider is only valid for learned routing")
            if not callable(alignment_provider):
                raise TypeError("alignment_provider must be callable")
        self._owned_alignment_provider = alignment_provider
        # the provider the next calls use: the owned one, or None (the built-in
        # alignment) inside bind_alignment_provider_for_capture(None, ...)
        self._active_alignment_provider = alignment_provider
        self._capture_lease: frozenset[tuple[int, int]] | None = None
        self._route_captures: dict[tuple[int, int], MoERouteCaptureBuffer] = {}
        self._route_capture_tensors: dict[tuple[int, int], tuple[torch.Tensor, ...]] = {}
        self._alignment_provider_poisoned = False
        self._alignment_provider_tensors = self._snapshot_provider_tensors(alignment_provider)
        if slots_per_shape < 1:
            raise ValueError("slots_per_shape must be positive")
        if buffer_donor is not None:
            if not isinstance(buffer_donor, TP4MoE) or buffer_donor is self:
                raise TypeError("buffer_donor must be a different TP4MoE")
            if buffer_donor.config != self.config or buffer_donor.device != self.device:
                raise ValueError("buffer_donor config/device differs")
            if buffer_donor.route_kind != self.route_kind:
                raise ValueError("buffer_donor route kind differs (input-ID storage shape)")
            needed = {(int(r), s) for r in global_row_shapes for s in range(slots_per_shape)}
            missing = needed - set(buffer_donor._buffers)
            if missing:
                raise ValueError(f"buffer_donor lacks registered shapes {sorted(missing)}")
            self._buffers = buffer_donor._buffers
        else:
            self._buffers: dict[tuple[int, int], _LayerBuffers] = {}
            for rows in global_row_shapes:
                for slot in range(slots_per_shape):
                    self._register_shape(int(rows), slot)
        self._validate_provider_storage()

    def _add_shared_fp8(self, flat: torch.Tensor, buffers: "_LayerBuffers", out: torch.Tensor) -> None:
        """output <- bf16(routed + shared(flat)) for an FP8-block shared expert
        (``moe_runtime.py:1860-1873``: shared_bf16_partial, then torch.add)."""

        if self._shared_fp8 is not None:
            ops.shared_fp8_add_into(flat, self._shared_fp8, clamp_limit=self.config.clamp_limit,
                                    out=out, workspace=buffers.shared_workspace)

    # ------------------------------------------------------------ buffers
    def _register_shape(self, rows: int, slot: int) -> None:
        cfg = self.config
        if rows <= 0:
            raise ValueError("MoE rows must be positive")
        key = (rows, slot)
        if key in self._buffers:
            return
        bs = ops.block_size_m(rows, cfg.topk, cfg.experts, 1 if self._marlin_input_dtype else 2)
        template = torch.empty(rows, cfg.topk, dtype=torch.int32, device=self.device)
        ws_fn = ops.experts_w4a8_workspace_bytes if self._marlin_input_dtype else ops.experts_workspace_bytes
        ws_bytes = ws_fn(rows, cfg.topk, cfg.hidden_size, cfg.intermediate_size, self._grouped_shared)
        self._buffers[key] = _LayerBuffers(
            workspace=torch.empty(ws_bytes, dtype=torch.uint8, device=self.device),
            logits=torch.empty(rows, cfg.experts, dtype=torch.float32, device=self.device),
            route_ids=torch.empty(rows, cfg.topk, dtype=torch.int32, device=self.device),
            route_weights=torch.empty(rows, cfg.topk, dtype=torch.float32, device=self.device),
            margin=torch.empty(rows, dtype=torch.float32, device=self.device),
            alignment=allocate_deterministic_moe_alignment(template, block_size=bs, num_experts=cfg.experts),
            block_size_m=bs,
            ready_event=torch.cuda.Event(blocking=False),
            gathered_input_ids=(
                torch.empty(rows, dtype=torch.int64, device=self.device)
                if self.route_kind == "hash" else None
            ),
            shared_workspace=(
                torch.empty(ops.shared_fp8_workspace_bytes(rows, cfg.hidden_size, cfg.intermediate_size),
                            dtype=torch.uint8, device=self.device)
                if self._shared_fp8 is not None else None
            ),
        )

    @property
    def registered_global_rows(self) -> tuple[int, ...]:
        return tuple(sorted({rows for rows, _ in self._buffers}))

    @property
    def registered_slots(self) -> dict[int, tuple[int, ...]]:
        return {
            rows: tuple(sorted(s for r, s in self._buffers if r == rows))
            for rows in self.registered_global_rows
        }

    @property
    def alignment_provider(self) -> Callable[..., object] | None:
        return self._owned_alignment_provider

    def block_size_for(self, rows: int, slot: int = 0) -> int:
        return self._buffers[(rows, slot)].block_size_m

    # ------------------------------------------------- alignment provider
    def _snapshot_provider_tensors(self, provider) -> tuple[torch.Tensor, ...]:
        """The provider's own storage (``storage_tensors()``, reference
        ``moe_runtime.py:631-666``): a tuple of non-empty, contiguous,
        gradient-free tensors on the layer's device, each the whole of its
        allocation, no two sharing one."""

        if provider is None:
            return ()
        lister = getattr(provider, "storage_tensors", None)
        if not callable(lister):
            raise TypeError("alignment_provider must expose a callable storage_tensors()")
        owned = lister()
        if not isinstance(owned, tuple):
            raise TypeError(f"alignment_provider.storage_tensors() returned {type(owned).__name__}, not a tuple")
        named = {f"alignment provider storage[{i}]": t for i, t in enumerate(owned)}
        for name, t in named.items():
            C.tensor(name, t, device=self.device, contiguous=True, no_grad=True, nonempty=True)
            C.owns_whole_storage(name, t)
        C.distinct_storages(named, what="alignment provider storage")
        return owned

    def _current_ratios(self) -> dict[str, torch.Tensor]:
        """The W4A16 prefill kernels' scale ratios, recomputed in place first
        if the resident scales changed since they were derived (a host-side
        check of the scales' storage and version; no device read)."""

        if self._ratio_kwargs:
            w13r, w2r = self.resident.scale_ratios()
            if w13r is not self._ratio_kwargs["w13r"] or w2r is not self._ratio_kwargs["w2r"]:
                self._ratio_kwargs = {"w13r": w13r, "w2r": w2r}
        return self._ratio_kwargs

    def _runtime_tensors(self) -> list[torch.Tensor]:
        tensors = [self.resident.w13_q, self.resident.w13_s, self.resident.w2_q, self.resident.w2_s,
                   self.gate.weight, *self._ratio_kwargs.values()]
        for b in self._buffers.values():
            tensors += [b.workspace, b.logits, b.route_ids, b.route_weights, b.margin,
                        b.alignment.sorted_token_ids, b.alignment.expert_ids,
                        b.alignment.num_tokens_post_padded]
        for owned in self._route_capture_tensors.values():
            tensors += list(owned)
        return tensors

    def _runtime_storage_pointers(self) -> set[int]:
        return {int(t.untyped_storage().data_ptr()) for t in self._runtime_tensors()}

    def _validate_provider_storage(self) -> None:
        if self._owned_alignment_provider is None:
            return
        observed = self._snapshot_provider_tensors(self._owned_alignment_provider)
        if len(observed) != len(self._alignment_provider_tensors) or any(
            a is not b for a, b in zip(observed, self._alignment_provider_tensors)
        ):
            raise ValueError("alignment provider storage tensor identity drifted")
        provider_ptrs = {int(t.untyped_storage().data_ptr()) for t in observed}
        if provider_ptrs & self._runtime_storage_pointers():
            raise ValueError("alignment provider storage aliases TP4MoE storage")

    def _poison_alignment_runtime(self) -> None:
        self._alignment_provider_poisoned = True
        for b in self._buffers.values():
            b.state = "poisoned"

    def _require_healthy(self) -> None:
        if self._alignment_provider_poisoned:
            raise RuntimeError("MoE alignment-provider lifecycle is poisoned; restart required")

    def _lifecycle(self, keys) -> dict[tuple[int, int], tuple[str, bool, int]]:
        return {key: (self._buffers[key].state, self._buffers[key].has_completion_event,
                      id(self._buffers[key].ready_event)) for key in keys}

    @contextmanager
    def bind_alignment_provider_for_capture(self, provider: Callable[..., object] | None, *,
                                            buffer_keys: Iterable[tuple[int, int]]) -> Iterator[None]:
        """Choose the alignment path (the owned provider, or None for the
        built-in alignment) for one fresh graph capture of the listed
        (rows, slot) buffers (reference ``moe_runtime.py:825-978``).

        On entry every slot must be free and each listed slot must have had
        its completion event reset; calls to unlisted slots are refused while
        the lease is held.  On exit the listed slots must be free with a new
        completion event (the captured call recorded it) and every other slot
        untouched; a failed capture must leave every slot as it was.  Any
        violation, and any change of the provider's storage, poisons the
        layer (RuntimeError; a restart is required).  Graphs captured before
        keep the path they captured.
        """

        if provider is not None and provider is not self._owned_alignment_provider:
            raise ValueError("the capture provider must be None or the layer's own alignment provider")
        self._require_healthy()
        if self._capture_lease is not None:
            raise RuntimeError("alignment-provider capture bindings cannot be nested")
        keys = tuple(buffer_keys)
        if not keys:
            raise ValueError("a capture binding needs at least one (rows, slot) key")
        for key in keys:
            if not (isinstance(key, tuple) and len(key) == 2
                    and all(isinstance(v, int) and not isinstance(v, bool) for v in key)):
                raise TypeError(f"capture binding keys are (rows, slot) integer pairs, got {key!r}")
            if key not in self._buffers:
                raise ValueError(f"capture binding key {key} is not a registered (rows, slot)")
        if len(set(keys)) != len(keys):
            raise ValueError("capture binding keys must be unique")
        busy = {k: b.state for k, b in self._buffers.items() if b.state != "free"}
        if busy:
            raise RuntimeError(f"a capture binding needs every slot free; busy: {busy}")
        stale = [k for k in keys if self._buffers[k].has_completion_event]
        if stale:
            raise RuntimeError(f"reset the completion events of {stale} before binding them for capture")
        before = self._lifecycle(self._buffers)
        try:
            self._validate_provider_storage()
        except Exception as exc:
            self._poison_alignment_runtime()
            raise RuntimeError("alignment-provider storage changed; restart required") from exc
        previous = self._active_alignment_provider
        self._active_alignment_provider = provider
        self._capture_lease = frozenset(keys)
        completed = False
        try:
            yield
            completed = True
        finally:
            self._active_alignment_provider = previous
            self._capture_lease = None
            after = self._lifecycle(self._buffers)
            problems = []
            for key in self._buffers:
                if completed and key in keys:
                    state, has_event, event = after[key]
                    if state != "free" or not has_event or event != before[key][2]:
                        problems.append(f"{key}: captured slot ended {state}, completion event {has_event}")
                elif after[key] != before[key]:
                    problems.append(f"{key}: lifecycle changed from {before[key]} to {after[key]}")
            try:
                self._validate_provider_storage()
            except Exception as exc:  # noqa: BLE001 - reported with the rest
                problems.append(f"provider storage: {exc}")
            if problems:
                self._poison_alignment_runtime()
                raise RuntimeError("capture binding left the layer inconsistent: " + "; ".join(problems))

    # ------------------------------------------------------ route capture
    @property
    def registered_route_capture_slots(self) -> dict[int, tuple[int, ...]]:
        rows = sorted({r for r, _ in self._route_captures})
        return {r: tuple(sorted(s for rr, s in self._route_captures if rr == r)) for r in rows}

    def register_route_capture(self, global_rows: int, slot: int = 0) -> MoERouteCaptureBuffer:
        """Allocate the stable route target of one (rows, slot) before a
        graph capture (reference ``moe_runtime.py:1017-1089``): every later
        call of that slot copies its effective route (ids, weights) there and
        adds one to the device generation, with no host read."""

        self._require_healthy()
        if self._capture_lease is not None:
            raise RuntimeError("route captures cannot be registered during a capture binding")
        if not all(isinstance(v, int) and not isinstance(v, bool) for v in (global_rows, slot)):
            raise TypeError("route capture rows and slot must be integers")
        key = (global_rows, slot)
        if key not in self._buffers:
            raise ValueError(f"route capture {key} has no registered buffers; registered={self.registered_slots}")
        if key in self._route_captures:
            raise RuntimeError(f"a route capture for {key} is already registered")
        shape = (global_rows, self.config.topk)
        owned = (torch.full(shape, -1, dtype=torch.int32, device=self.device),
                 torch.zeros(shape, dtype=torch.float32, device=self.device),
                 torch.zeros(1, dtype=torch.int64, device=self.device))
        capture = MoERouteCaptureBuffer(global_rows=global_rows, slot=slot, owner_id=id(self), ids=owned[0],
                                        weights=owned[1], generation=owned[2],
                                        tensor_pointers=tuple(int(t.data_ptr()) for t in owned))
        self._route_captures[key] = capture
        self._route_capture_tensors[key] = owned
        try:
            self._check_route_capture(key, capture)
        except BaseException:
            del self._route_captures[key], self._route_capture_tensors[key]
            raise
        try:
            self._validate_provider_storage()
        except BaseException as exc:
            del self._route_captures[key], self._route_capture_tensors[key]
            self._poison_alignment_runtime()
            raise RuntimeError("registering a route capture broke the provider storage; restart required") from exc
        return capture

    def _check_route_capture(self, key: tuple[int, int], capture: MoERouteCaptureBuffer) -> None:
        """The registered capture object and its tensors are unchanged and
        share storage with nothing else of the layer."""

        if not isinstance(capture, MoERouteCaptureBuffer):
            raise TypeError("route capture has the wrong type")
        owned = self._route_capture_tensors.get(key)
        if owned is None or self._route_captures.get(key) is not capture:
            raise ValueError(f"route capture {key} is not the one registered")
        if (capture.owner_id, capture.global_rows, capture.slot) != (id(self), *key):
            raise ValueError(f"route capture {key} belongs to another layer or slot")
        shape = (key[0], self.config.topk)
        expected = (("ids", capture.ids, shape, torch.int32), ("weights", capture.weights, shape, torch.float32),
                    ("generation", capture.generation, (1,), torch.int64))
        for (name, t, want, dtype), mine in zip(expected, owned):
            if t is not mine:
                raise ValueError(f"route capture {key}: {name} was replaced")
            C.tensor(f"route capture {name}", t, shape=want, dtype=dtype, device=self.device, contiguous=True,
                     no_grad=True, dtype_error=ValueError)
        if tuple(int(t.data_ptr()) for t in owned) != capture.tensor_pointers:
            raise ValueError(f"route capture {key}: storage moved")
        mine = {int(t.untyped_storage().data_ptr()) for t in owned}
        if len(mine) != 3:
            raise ValueError(f"route capture {key}: its tensors share storage")
        others = [t for k, ts in self._route_capture_tensors.items() if k != key for t in ts]
        for b in self._buffers.values():
            others += [b.workspace, b.route_ids, b.route_weights, b.alignment.sorted_token_ids,
                       b.alignment.expert_ids, b.alignment.num_tokens_post_padded]
        if mine & {int(t.untyped_storage().data_ptr()) for t in others}:
            raise ValueError(f"route capture {key}: storage aliases another buffer of the layer")

    def route_capture_buffer(self, global_rows: int, slot: int = 0) -> MoERouteCaptureBuffer:
        key = (global_rows, slot)
        capture = self._route_captures.get(key)
        if capture is None:
            raise ValueError(f"no route capture is registered for {key}")
        self._check_route_capture(key, capture)
        return capture

    def snapshot_route_capture(self, global_rows: int, slot: int = 0, *,
                               expected_generation: int) -> MoERouteCaptureEvidence:
        """A host copy of the capture buffer (reference
        ``moe_runtime.py:1190-1227``); synchronises, so it belongs outside
        replay and timed regions.  The device generation must equal
        ``expected_generation`` before and after the copy."""

        if isinstance(expected_generation, bool) or not isinstance(expected_generation, int) \
                or expected_generation <= 0:
            raise ValueError("expected_generation must be a positive integer")
        capture = self.route_capture_buffer(global_rows, slot)
        seen = int(capture.generation.item())
        if seen == 0:
            raise RuntimeError("the route capture has not recorded a route yet")
        if seen != expected_generation:
            raise RuntimeError(f"route capture generation is {seen}, expected {expected_generation}")
        ids = capture.ids.detach().cpu().clone()
        weights = capture.weights.detach().cpu().clone()
        if int(capture.generation.item()) != expected_generation:
            raise RuntimeError("the route capture changed while it was being copied")
        return MoERouteCaptureEvidence(global_rows=global_rows, slot=slot, ids=ids, weights=weights,
                                       generation=seen, device_tensor_pointers=capture.tensor_pointers,
                                       route_digest=_tensor_digest(ids, weights))

    def reset_route_capture_generation(self, global_rows: int, slot: int = 0) -> None:
        """Zero the device generation in place (after graph setup / warm-up)."""

        self.route_capture_buffer(global_rows, slot).generation.zero_()

    def _capture_route(self, key: tuple[int, int], weights: torch.Tensor,
                       ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Copy the effective route into the registered capture buffer on the
        current stream and return the buffer's tensors, which the rest of the
        call then uses (reference ``moe_runtime.py:1237-1283``)."""

        for k, cap in self._route_captures.items():
            self._check_route_capture(k, cap)
        capture = self._route_captures[key]
        want = (key[0], self.config.topk)
        C.tensor("effective route ids", ids, shape=want, dtype=torch.int32, device=self.device, contiguous=True,
                 dtype_error=ValueError)
        C.tensor("effective route weights", weights, shape=want, dtype=torch.float32, device=self.device,
                 contiguous=True, dtype_error=ValueError)
        sources = {int(ids.untyped_storage().data_ptr()), int(weights.untyped_storage().data_ptr())}
        if len(sources) != 2:
            raise ValueError("effective route ids and weights share storage")
        targets = {int(t.untyped_storage().data_ptr()) for ts in self._route_capture_tensors.values() for t in ts}
        if sources & targets:
            raise ValueError("the effective route already lives in a route capture buffer")
        capture.ids.copy_(ids)
        capture.weights.copy_(weights)
        capture.generation.add_(1)
        return capture.weights, capture.ids

    # ----------------------------------------------------- lifecycle
    def slot_completion_status(self, global_rows: int, slot: int) -> dict[str, Any]:
        key = (global_rows, slot)
        if key not in self._buffers:
            raise ValueError(f"global row/slot {key} was not pre-registered")
        b = self._buffers[key]
        return {"state": b.state, "has_completion_event": b.has_completion_event}

    def reset_free_slot_completion_event(self, global_rows: int, slot: int) -> None:
        self._require_healthy()
        if self._capture_lease is not None:
            raise RuntimeError("slot completion events cannot be reset during a capture binding")
        key = (global_rows, slot)
        if key not in self._buffers:
            raise ValueError(f"global row/slot {key} was not pre-registered")
        b = self._buffers[key]
        if b.state != "free":
            raise RuntimeError(f"MoE buffer slot {key} is not free")
        b.ready_event = torch.cuda.Event(blocking=False)
        b.has_completion_event = False

    def enable_collective_overlap(self, blocks: int) -> None:
        """No collectives at world size 1: accepted and recorded, never engaged."""

        if not isinstance(blocks, int) or blocks < 0:
            raise ValueError("blocks must be a non-negative integer")
        self._overlap_blocks = blocks

    @contextmanager
    def observe_route_tensors(self, *, capture_local_input: bool = False) -> Iterator[list[MoERouteTensors]]:
        """Collect the route tensors of every call inside the block (reference
        ``moe_runtime.py:1318-1335``), optionally with a copy of the input."""

        C.boolean("capture_local_input", capture_local_input)
        if self._route_tensor_observer is not None:
            raise RuntimeError("route tensor observation is already active")
        self._route_tensor_observer = collected = []
        self._route_observer_captures_local_input = capture_local_input
        try:
            yield collected
        finally:
            self._route_tensor_observer = None
            self._route_observer_captures_local_input = False

    # ------------------------------------------------------- forward
    def __call__(
        self,
        hidden_local: torch.Tensor,
        *,
        input_ids_local: torch.Tensor | None = None,
        route_override: MoERouteOverride | None = None,
        router_logits: torch.Tensor | None = None,
        local_step: Callable[[str, Callable[[], Any]], Any] | None = None,
        slot: int = 0,
        collect_trace: bool = True,
        collect_stage_digests: bool = False,
        stage_marker: Callable[[str], None] | None = None,
    ) -> tuple[torch.Tensor, MoETrace | None]:
        """One MoE layer forward (``moe_runtime.py:1565-1947``).

        ``router_logits`` (fp32 [rows, E], optional) replaces the gate GEMM for
        callers that already hold the logits; selection, weights and margin are
        still computed from them with the configured score function.
        """

        cfg = self.config

        def run_local(name: str, fn: Callable[[], Any]) -> Any:
            return fn() if local_step is None else local_step(name, fn)

        def mark(name: str) -> None:
            if stage_marker is not None:
                stage_marker(name)

        def prepare_input():
            if hidden_local.ndim != 3 or hidden_local.shape[-1] != cfg.hidden_size:
                raise ValueError("MoE input must have shape [local_batch, sequence, hidden]")
            if hidden_local.dtype != torch.bfloat16 or hidden_local.device != self.device:
                raise ValueError("MoE input must use the configured device and BF16")
            local_ids = None
            if self.route_kind == "learned":
                if input_ids_local is not None:
                    raise ValueError("learned routing forbids input_ids_local")
            else:
                if route_override is not None:
                    raise ValueError("hash routing forbids route_override")
                if router_logits is not None:
                    raise ValueError("hash routing computes its own logits")
                if not isinstance(input_ids_local, torch.Tensor):
                    raise ValueError("hash routing requires input_ids_local")
                if tuple(input_ids_local.shape) != tuple(hidden_local.shape[:-1]):
                    raise ValueError("input_ids_local shape must match hidden local row axes")
                if input_ids_local.dtype != torch.int64 or input_ids_local.device != self.device:
                    raise ValueError("input_ids_local must be int64 on the configured device")
                if not input_ids_local.is_contiguous():
                    raise ValueError("input_ids_local must be contiguous")
                local_ids = input_ids_local.view(-1)
                # A token id outside the table routes to expert -1 on the device:
                # the alignment then reports a negative padded count and every
                # output of the call is NaN.  The host-side range check costs a
                # device-to-host read per call, so it runs only when the caller
                # asks for it (check_hash_token_ids), and never under capture.
                if self.check_hash_token_ids and (
                        local_ids.device.type != "cuda" or not torch.cuda.is_current_stream_capturing()):
                    C.ids_below("input_ids_local", local_ids, int(self.gate.tid2eid.shape[0]))
            shape = tuple(hidden_local.shape)
            flat = hidden_local.reshape(-1, cfg.hidden_size).contiguous()
            rows = flat.shape[0]
            override = None
            if route_override is not None:
                override = _snapshot_route_override(route_override, rows=rows, config=cfg, device=self.device)
            if router_logits is not None:
                if tuple(router_logits.shape) != (rows, cfg.experts) or router_logits.dtype != torch.float32:
                    raise ValueError(f"router_logits must be fp32 [{rows}, {cfg.experts}]")
                if router_logits.device != self.device or not router_logits.is_contiguous():
                    raise ValueError("router_logits must be contiguous on the configured device")
            key = (rows, slot)
            if key not in self._buffers:
                raise ValueError(
                    f"global row/slot {key} was not pre-registered; registered={self.registered_slots}"
                )
            self._require_healthy()
            if self._capture_lease is not None and key not in self._capture_lease:
                raise RuntimeError(f"MoE buffer slot {key} is outside the active graph-capture binding")
            b = self._buffers[key]
            if b.state != "free":
                raise RuntimeError(
                    f"MoE buffer slot {key} is {b.state}; worker restart is required after a poisoned slot"
                )
            if self.device.type != "cuda":
                raise ValueError("this TP4MoE was built on the CPU for host-side checks; it computes on a GPU")
            return shape, flat, local_ids, override, b

        shape, flat, local_ids, override, buffers = run_local("prepare MoE input", prepare_input)
        buffers.state = "in_flight"
        if buffers.has_completion_event:
            torch.cuda.current_stream(self.device).wait_event(buffers.ready_event)
        try:
            self.overlap_stats["sequential_calls"] += 1
            self.overlap_stats["sequential_rows"] += int(flat.shape[0])
            mark("moe_inputs_ready")
            mark("moe_hidden_all_gather_done")
            if local_ids is not None and buffers.gathered_input_ids is not None:
                buffers.gathered_input_ids.copy_(local_ids)
            mark("moe_ids_all_gather_done")

            # the call's result: a fresh owning tensor that the combine writes
            # directly (the reference returns an owning clone of its buffer)
            output = torch.empty((flat.shape[0], cfg.hidden_size), dtype=torch.bfloat16, device=self.device)

            def compute_partial():
                route_source = "native"
                margin = None
                a = buffers.alignment
                capture_key = (flat.shape[0], slot)
                fused = (
                    self.route_kind == "learned"
                    and override is None
                    and self._active_alignment_provider is None
                    and self._route_tensor_observer is None
                    and capture_key not in self._route_captures
                    and stage_marker is None
                )
                if self.route_kind == "learned" and router_logits is None:
                    ops.gate_logits_into(flat, self._gate_weight, buffers.logits)
                logits = router_logits if router_logits is not None else buffers.logits
                if fused and self._marlin_input_dtype is not None:
                    # route -> align (x quantised beside it) -> W4A8 experts -> combine
                    ops.layer_w4a8_into(
                        flat, logits, self._gate_bias, topk=cfg.topk, score_func=cfg.score_func,
                        route_scale=cfg.route_scale, w13q=self.resident.w13_q,
                        w13s=self.resident.w13_s, w2q=self.resident.w2_q, w2s=self.resident.w2_s,
                        experts=cfg.experts, inter=cfg.intermediate_size,
                        has_shared=self._grouped_shared, clamp_limit=cfg.clamp_limit,
                        block_size=buffers.block_size_m, ids=buffers.route_ids,
                        weights=buffers.route_weights, margin=buffers.margin,
                        sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
                        num_tokens_post_padded=a.num_tokens_post_padded, out=output,
                        workspace=buffers.workspace, mxfp4=self._mxfp4,
                    )
                    self._add_shared_fp8(flat, buffers, output)
                    return buffers.route_weights, buffers.route_ids, buffers.margin, {}
                if fused:
                    # route -> align -> experts -> combine in one C-ABI call
                    ops.layer_w4a16_into(
                        flat, logits, self._gate_bias, topk=cfg.topk, score_func=cfg.score_func,
                        route_scale=cfg.route_scale, w13q=self.resident.w13_q,
                        w13s=self.resident.w13_s, w2q=self.resident.w2_q, w2s=self.resident.w2_s,
                        **self._current_ratios(), experts=cfg.experts, inter=cfg.intermediate_size,
                        has_shared=self._grouped_shared, clamp_limit=cfg.clamp_limit,
                        block_size=buffers.block_size_m, ids=buffers.route_ids,
                        weights=buffers.route_weights, margin=buffers.margin,
                        sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
                        num_tokens_post_padded=a.num_tokens_post_padded, out=output,
                        workspace=buffers.workspace, mxfp4=self._mxfp4,
                    )
                    self._add_shared_fp8(flat, buffers, output)
                    return buffers.route_weights, buffers.route_ids, buffers.margin, {}
                sel_ids = sel_scores = None
                if self.route_kind == "hash":
                    ops.gate_logits_into(flat, self._gate_weight, buffers.logits)
                    ops.route_hash_into(
                        buffers.logits, self.gate.tid2eid, buffers.gathered_input_ids,
                        route_scale=cfg.route_scale, ids=buffers.route_ids,
                        weights=buffers.route_weights,
                    )
                    route_ids, route_weights = buffers.route_ids, buffers.route_weights
                else:
                    if self._route_tensor_observer is not None:
                        depth = min(cfg.topk + 1, cfg.experts)
                        sel_ids = torch.empty(flat.shape[0], depth, dtype=torch.int32, device=self.device)
                        sel_scores = torch.empty(flat.shape[0], depth, dtype=torch.float32, device=self.device)
                    ops.route_topk_into(
                        logits, self._gate_bias, topk=cfg.topk, score_func=cfg.score_func,
                        route_scale=cfg.route_scale, ids=buffers.route_ids,
                        weights=buffers.route_weights, margin=buffers.margin,
                        selection_ids=sel_ids, selection_scores=sel_scores,
                    )
                    margin = buffers.margin
                    route_ids, route_weights = buffers.route_ids, buffers.route_weights
                    if override is not None:
                        route_ids, route_weights = override
                        route_source = "explicit_global"
                mark("moe_route_done")
                if self._route_tensor_observer is not None:
                    self._route_tensor_observer.append(
                        MoERouteTensors(
                            weights=route_weights, ids=route_ids, margin=margin,
                            selection_ids=sel_ids, selection_scores=sel_scores,
                            local_input=flat.detach().clone() if self._route_observer_captures_local_input else None,
                            gate_logits=logits if self.route_kind == "learned" else buffers.logits,
                            route_source=route_source,
                        )
                    )
                if capture_key in self._route_captures:
                    route_weights, route_ids = self._capture_route(capture_key, route_weights, route_ids)
                provider = self._active_alignment_provider
                if provider is None:
                    # the experts workspace is idle until the experts launches, which
                    # follow on the same stream: it holds the split alignment's scratch
                    ops.align_into(
                        route_ids, block_size=buffers.block_size_m, num_experts=cfg.experts,
                        sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
                        num_tokens_post_padded=a.num_tokens_post_padded,
                        workspace=buffers.workspace,
                    )
                else:
                    try:
                        aligned = provider(route_ids, block_size=buffers.block_size_m,
                                           num_experts=cfg.experts, output=a, slot=slot)
                    except BaseException:
                        self._poison_alignment_runtime()
                        raise
                    if aligned is not a:
                        self._poison_alignment_runtime()
                        raise RuntimeError("alignment provider must return the caller-owned output")
                if self._mxfp4:
                    experts_into = ops.experts_w4a8_mxfp4_into if self._marlin_input_dtype else ops.experts_mxfp4_into
                elif self._marlin_input_dtype:
                    experts_into = ops.experts_w4a8_into
                else:
                    experts_into = ops.experts_w4a16_into
                experts_into(
                    flat, w13q=self.resident.w13_q, w13s=self.resident.w13_s,
                    w2q=self.resident.w2_q, w2s=self.resident.w2_s, **self._current_ratios(), experts=cfg.experts,
                    inter=cfg.intermediate_size, has_shared=self._grouped_shared,
                    route_weights=route_weights, sorted_token_ids=a.sorted_token_ids,
                    expert_ids=a.expert_ids, num_tokens_post_padded=a.num_tokens_post_padded,
                    block_size=buffers.block_size_m, clamp_limit=cfg.clamp_limit,
                    out=output, workspace=buffers.workspace,
                )
                # routed experts, shared expert and the add run in the same fused launch chain
                # (an FP8-block shared expert as dense linears that add into the routed sum)
                mark("moe_routed_done")
                self._add_shared_fp8(flat, buffers, output)
                mark("moe_shared_done")
                mark("moe_combine_done")
                digests = {}
                if collect_stage_digests:
                    digests = {
                        "gathered_input": _tensor_digest(flat),
                        "combined_partial": _tensor_digest(output),
                    }
                return route_weights, route_ids, margin, digests

            route_weights, route_ids, margin, digests = run_local("compute MoE partial", compute_partial)
            mark("moe_reduce_scatter_done")

            def finish():
                out = output.view(shape)
                trace = None
                if collect_trace:
                    if collect_stage_digests:
                        digests["reduce_scatter_output"] = _tensor_digest(output)
                    trace = MoETrace(
                        local_input_shape=shape,
                        gathered_shape=tuple(flat.shape),
                        partial_shape=tuple(output.shape),
                        local_output_shape=tuple(out.shape),
                        route_ids_row_zero=tuple(int(v) for v in route_ids[0].cpu()),
                        route_weights_row_zero=tuple(float(v) for v in route_weights[0].cpu()),
                        route_margin_min=None if margin is None else float(margin.min().item()),
                        route_digest=_tensor_digest(route_ids, route_weights),
                        stage_digests=digests,
                        buffer_slot=slot,
                        route_source="explicit_global" if override is not None else "native",
                    )
                buffers.ready_event.record(torch.cuda.current_stream(self.device))
                buffers.has_completion_event = True
                buffers.state = "free"
                return out, trace

            result = run_local("finalize MoE trace", finish)
            mark("moe_finalize_done")
            return result
        except BaseException:
            buffers.state = "poisoned"
            raise

    def forward_tensor(
        self,
        hidden_local: torch.Tensor,
        *,
        input_ids_local: torch.Tensor | None = None,
        route_override: MoERouteOverride | None = None,
        router_logits: torch.Tensor | None = None,
        slot: int = 0,
        stage_marker: Callable[[str], None] | None = None,
    ) -> torch.Tensor:
        """Owning output without host-side trace extraction (``moe_runtime.py:1949-1970``)."""

        out, trace = self(
            hidden_local,
            input_ids_local=input_ids_local,
            route_override=route_override,
            router_logits=router_logits,
            slot=slot,
            collect_trace=False,
            stage_marker=stage_marker,
        )
        if trace is not None:
            raise AssertionError("trace-free MoE path unexpectedly produced a trace")
        return out


MoELayer = TP4MoE

__all__ = [
    "FLASH_CONFIG",
    "MoELayer",
    "MoERouteCaptureBuffer",
    "MoERouteCaptureEvidence",
    "MoERouteOverride",
    "MoERouteTensors",
    "MoETrace",
    "ResidentGateWeights",
    "TP4MoE",
    "TP4MoEConfig",
]
