"""Fixed-geometry MoE alignment for the B240 decode graph.

Drop-in for ``runtime/dsv4_direct/fixed_moe_align.py``: the same constants,
plan and workspace dataclasses, the alignment-provider class that
``TP4MoE(alignment_provider=...)`` and ``bind_alignment_provider_for_capture``
accept (``storage_tensors()``, ``provider_identity()``, the provider call),
the cold-path allocator, the metadata / non-alias validator and the hot
wrapper ``fixed_b240_moe_align_block8``, with the reference's exception
classes.  The geometry is fixed: route ids ``int32 [240, 6]``, 256 experts,
blocks of 8 routes, capacity ``1440 + 256 * 7 = 3232`` slots in 404 blocks.

The layout (expert-major, ascending flat index ``t*6 + j`` inside each
expert, every expert run padded with the sentinel 1440 to a multiple of 8,
the sentinel past the padded total, ``-1`` for blocks past it) is written by
the HIP alignment kernel (``dsv4moe_align``: one workgroup, LDS histogram and
ballot-ranked stable scatter, one launch), the same kernel as the general
alignment; it is stream-ordered, performs no host read and is graph
capturable.  The reference's four Triton launches count into the caller's
``counts_and_offsets`` workspace; here the counts live in LDS, and the
workspace tensor is kept as the provider's owned storage (its contract with
``TP4MoE``) without being written.

The reference module's CPU oracle ``fixed_b240_alignment_oracle`` is not part
of this package: the product computes on the GPU only.  Its restatement for
tests is ``oracle.moe_align_bruteforce`` at the B240 geometry.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable

import torch

from . import contracts as C
from . import ops
from .deterministic_moe_align import DeterministicMoEAlignment

FIXED_ROWS = 240
FIXED_TOPK = 6
FIXED_NUM_ASSIGNMENTS = FIXED_ROWS * FIXED_TOPK
FIXED_NUM_EXPERTS = 256
FIXED_BLOCK_SIZE = 8
FIXED_SENTINEL = FIXED_NUM_ASSIGNMENTS
FIXED_MAX_PADDED_TOKENS = FIXED_NUM_ASSIGNMENTS + FIXED_NUM_EXPERTS * (FIXED_BLOCK_SIZE - 1)
FIXED_MAX_BLOCKS = FIXED_MAX_PADDED_TOKENS // FIXED_BLOCK_SIZE
WORKSPACE_CAPACITY = 512


@dataclass(frozen=True)
class FixedB240AlignmentPlan:
    """The fixed geometry (reference ``fixed_moe_align.py:44-55``).
    ``launch_count`` is this build's: one HIP launch."""

    route_shape: tuple[int, int] = (FIXED_ROWS, FIXED_TOPK)
    num_assignments: int = FIXED_NUM_ASSIGNMENTS
    num_experts: int = FIXED_NUM_EXPERTS
    block_size: int = FIXED_BLOCK_SIZE
    sentinel: int = FIXED_SENTINEL
    max_padded_tokens: int = FIXED_MAX_PADDED_TOKENS
    max_blocks: int = FIXED_MAX_BLOCKS
    workspace_capacity: int = WORKSPACE_CAPACITY
    launch_count: int = 1


FIXED_B240_ALIGNMENT_PLAN = FixedB240AlignmentPlan()


@dataclass(frozen=True)
class FixedB240AlignmentWorkspace:
    """Caller-owned int32 [512] scratch of one graph slot (reference
    ``:61-64``)."""

    counts_and_offsets: torch.Tensor


def fixed_b240_max_padded_tokens() -> int:
    """The fixed capacity including worst-case padding: 3232."""

    return FIXED_MAX_PADDED_TOKENS


def _new_workspace(device: torch.device) -> FixedB240AlignmentWorkspace:
    return FixedB240AlignmentWorkspace(
        counts_and_offsets=torch.zeros(WORKSPACE_CAPACITY, dtype=torch.int32, device=device))


class FixedB240MoEAlignmentProvider:
    """An alignment provider owning one fixed workspace per (240, slot) graph
    slot (reference ``:67-155``)."""

    def __init__(self, *, device: torch.device, global_row_shapes: Iterable[int], slots_per_shape: int,
                 route_kind: str) -> None:
        device = torch.device(device)
        shapes = tuple(global_row_shapes)
        if shapes != (FIXED_ROWS,):
            raise ValueError(f"fixed B240 alignment serves global_row_shapes=({FIXED_ROWS},), got {shapes}")
        if isinstance(slots_per_shape, bool) or not isinstance(slots_per_shape, int) or slots_per_shape < 1:
            raise ValueError(f"fixed B240 alignment: slots_per_shape must be a positive int, got {slots_per_shape!r}")
        if route_kind != "learned":
            raise ValueError(f"fixed B240 alignment serves learned routing only, not {route_kind!r}")
        self.device = device
        self.global_row_shapes = shapes
        self.slots_per_shape = slots_per_shape
        self.route_kind = route_kind
        self._workspaces = {(FIXED_ROWS, slot): _new_workspace(device) for slot in range(slots_per_shape)}

    def storage_tensors(self) -> tuple[torch.Tensor, ...]:
        return tuple(self._workspaces[(FIXED_ROWS, s)].counts_and_offsets for s in range(self.slots_per_shape))

    @property
    def resident_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.storage_tensors())

    def provider_identity(self) -> dict[str, object]:
        plan = FIXED_B240_ALIGNMENT_PLAN
        return {
            "provider": "direct_fixed_b240_moe_alignment",
            "route_kind": self.route_kind,
            "global_row_shapes": list(self.global_row_shapes),
            "slots_per_shape": self.slots_per_shape,
            "route_shape": list(plan.route_shape),
            "num_experts": plan.num_experts,
            "block_size": plan.block_size,
            "workspace_capacity": plan.workspace_capacity,
            "launch_count": plan.launch_count,
        }

    def __call__(self, topk_ids: torch.Tensor, *, block_size: int, num_experts: int,
                 output: DeterministicMoEAlignment, slot: int) -> DeterministicMoEAlignment:
        if block_size != FIXED_BLOCK_SIZE or num_experts != FIXED_NUM_EXPERTS:
            raise ValueError(f"fixed B240 alignment is block {FIXED_BLOCK_SIZE} over {FIXED_NUM_EXPERTS} experts; "
                             f"asked for block {block_size} over {num_experts}")
        if isinstance(slot, bool) or not isinstance(slot, int):
            raise TypeError(f"fixed B240 alignment: slot must be an int, got {type(slot).__name__}")
        key = (FIXED_ROWS, slot)
        if key not in self._workspaces:
            raise ValueError(f"fixed B240 alignment: slot {slot} is not registered")
        if not isinstance(topk_ids, torch.Tensor) or topk_ids.device != self.device:
            raise ValueError(f"fixed B240 alignment: route ids must be on {self.device}")
        return fixed_b240_moe_align_block8(topk_ids, output=output, workspace=self._workspaces[key])


def _validate_route_metadata(topk_ids: torch.Tensor) -> None:
    if not isinstance(topk_ids, torch.Tensor):
        raise TypeError(f"topk_ids: expected a tensor, got {type(topk_ids).__name__}")
    if tuple(topk_ids.shape) != FIXED_B240_ALIGNMENT_PLAN.route_shape:
        raise ValueError(f"topk_ids: the fixed shape is {list(FIXED_B240_ALIGNMENT_PLAN.route_shape)}, "
                         f"got {list(topk_ids.shape)}")
    if topk_ids.dtype != torch.int32:
        raise TypeError(f"topk_ids: the fixed ABI is int32, got {topk_ids.dtype}")
    if not topk_ids.is_contiguous():
        raise ValueError("topk_ids must be contiguous")


def allocate_fixed_b240_alignment(topk_ids: torch.Tensor
                                  ) -> tuple[DeterministicMoEAlignment, FixedB240AlignmentWorkspace]:
    """Output and workspace for one slot, allocated on a cold path."""

    _validate_route_metadata(topk_ids)
    dev = topk_ids.device
    output = DeterministicMoEAlignment(
        sorted_token_ids=torch.empty(FIXED_MAX_PADDED_TOKENS, dtype=torch.int32, device=dev),
        expert_ids=torch.empty(FIXED_MAX_BLOCKS, dtype=torch.int32, device=dev),
        num_tokens_post_padded=torch.empty(1, dtype=torch.int32, device=dev),
    )
    return output, _new_workspace(dev)


def validate_fixed_b240_alignment_tensors(topk_ids: torch.Tensor, *, output: DeterministicMoEAlignment,
                                          workspace: FixedB240AlignmentWorkspace) -> torch.device:
    """Metadata and non-alias checks without reading the routes (reference
    ``:189-234``): TypeError for a wrong container, a non-tensor or non-int32
    route ids; ValueError for every shape, dtype, device, layout or aliasing
    mismatch.  Returns the device."""

    _validate_route_metadata(topk_ids)
    if not isinstance(output, DeterministicMoEAlignment):
        raise TypeError(f"output: expected DeterministicMoEAlignment, got {type(output).__name__}")
    if not isinstance(workspace, FixedB240AlignmentWorkspace):
        raise TypeError(f"workspace: expected FixedB240AlignmentWorkspace, got {type(workspace).__name__}")
    fields = {
        "topk_ids": (topk_ids, (FIXED_ROWS, FIXED_TOPK)),
        "output.sorted_token_ids": (output.sorted_token_ids, (FIXED_MAX_PADDED_TOKENS,)),
        "output.expert_ids": (output.expert_ids, (FIXED_MAX_BLOCKS,)),
        "output.num_tokens_post_padded": (output.num_tokens_post_padded, (1,)),
        "workspace.counts_and_offsets": (workspace.counts_and_offsets, (WORKSPACE_CAPACITY,)),
    }
    for name, (t, shape) in fields.items():
        C.tensor(name, t, shape=shape, dtype=torch.int32, dtype_error=ValueError, device=topk_ids.device,
                 contiguous=True)
    C.distinct_storages({name: t for name, (t, _) in fields.items()}, what="fixed B240 route, output and workspace")
    return topk_ids.device


def fixed_b240_moe_align_block8(topk_ids: torch.Tensor, *, output: DeterministicMoEAlignment,
                                workspace: FixedB240AlignmentWorkspace) -> DeterministicMoEAlignment:
    """The exact expert-major layout into the caller's fixed storage (one HIP
    launch on the current stream, no host read, no allocation).  A route id
    outside [0, 256) is reported on the device as ``num_tokens_post_padded =
    -1``, which the expert kernels turn into NaN outputs."""

    device = validate_fixed_b240_alignment_tensors(topk_ids, output=output, workspace=workspace)
    if device.type != "cuda":
        raise RuntimeError("fixed B240 alignment runs on the GPU; the tensors are on the CPU")
    ops.align_into(topk_ids, block_size=FIXED_BLOCK_SIZE, num_experts=FIXED_NUM_EXPERTS,
                   sorted_token_ids=output.sorted_token_ids, expert_ids=output.expert_ids,
                   num_tokens_post_padded=output.num_tokens_post_padded)
    return output


__all__ = [
    "FIXED_BLOCK_SIZE",
    "FIXED_B240_ALIGNMENT_PLAN",
    "FIXED_MAX_BLOCKS",
    "FIXED_MAX_PADDED_TOKENS",
    "FIXED_NUM_ASSIGNMENTS",
    "FIXED_NUM_EXPERTS",
    "FIXED_ROWS",
    "FIXED_SENTINEL",
    "FIXED_TOPK",
    "FixedB240AlignmentPlan",
    "FixedB240AlignmentWorkspace",
    "FixedB240MoEAlignmentProvider",
    "WORKSPACE_CAPACITY",
    "allocate_fixed_b240_alignment",
    "fixed_b240_max_padded_tokens",
    "fixed_b240_moe_align_block8",
    "validate_fixed_b240_alignment_tensors",
]
