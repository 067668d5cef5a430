"""Deterministic fixed-capacity MoE alignment on the HIP align kernel.

Drop-in for ``runtime/dsv4_direct/deterministic_moe_align.py``: same dataclass,
same capacity rule, the same exception classes for bad arguments, same output
layout (the public ``moe_align_block_size`` ABI).  The layout is computed by one workgroup of the
HIP kernel ``align_kernel`` (ballot-ranked stable permutation), or for many
ids by the chunk-count and chunk-scatter kernels over a temporary scratch
tensor (in place of the reference's torch temporaries), with no host read of
route-dependent data.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import contracts as C
from . import ops


@dataclass(frozen=True)
class DeterministicMoEAlignment:
    sorted_token_ids: torch.Tensor
    expert_ids: torch.Tensor
    num_tokens_post_padded: torch.Tensor


def max_padded_tokens(num_assignments: int, num_experts: int, block_size: int) -> int:
    """Fixed capacity (``deterministic_moe_align.py:17-32``)."""

    a = C.positive_int("num_assignments", num_assignments)
    e = C.positive_int("num_experts", num_experts)
    bs = C.positive_int("block_size", block_size)
    # every expert run padded by at most bs - 1; with fewer assignments than
    # experts at most `a` runs exist, each at most one block long
    padded_runs = a + e * (bs - 1)
    return min(padded_runs, a * bs) if a < e else padded_runs


def allocate_deterministic_moe_alignment(
    topk_ids: torch.Tensor, *, block_size: int, num_experts: int
) -> DeterministicMoEAlignment:
    """Caller-owned output storage (``deterministic_moe_align.py:35-55``)."""

    capacity = _validate_metadata(topk_ids, block_size=block_size, num_experts=num_experts)
    return DeterministicMoEAlignment(
        sorted_token_ids=torch.empty(capacity, dtype=torch.int32, device=topk_ids.device),
        expert_ids=torch.empty(-(-capacity // block_size), dtype=torch.int32, device=topk_ids.device),
        num_tokens_post_padded=torch.empty(1, dtype=torch.int32, device=topk_ids.device),
    )


def deterministic_moe_align_block_size(
    topk_ids: torch.Tensor,
    *,
    block_size: int,
    num_experts: int,
    output: DeterministicMoEAlignment | None = None,
) -> DeterministicMoEAlignment:
    """Expert-major alignment with ascending flat indices
    (``deterministic_moe_align.py:58-133``).

    ``sorted_token_ids`` stores row-major indices into ``topk_ids.flatten()``;
    unused rows hold the sentinel ``topk_ids.numel()``; every active block of
    ``expert_ids`` names one expert, the rest are -1.  An out-of-range route id
    is reported as ``num_tokens_post_padded == -1`` (the kernel writes nothing
    else), since ids are never read on the host.
    """

    capacity = _validate_metadata(topk_ids, block_size=block_size, num_experts=num_experts)
    if topk_ids.device.type != "cuda":
        raise ValueError("deterministic_moe_align_block_size runs on the GPU; got a CPU tensor")
    if output is None:
        output = allocate_deterministic_moe_alignment(
            topk_ids, block_size=block_size, num_experts=num_experts
        )
    _validate_output(output, topk_ids=topk_ids, block_size=block_size, capacity=capacity)
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    scratch_bytes = ops.align_workspace_bytes(ids.shape[0], ids.shape[1], num_experts)
    ops.align_into(
        ids,
        block_size=block_size,
        num_experts=num_experts,
        sorted_token_ids=output.sorted_token_ids,
        expert_ids=output.expert_ids,
        num_tokens_post_padded=output.num_tokens_post_padded,
        workspace=(torch.empty(scratch_bytes, dtype=torch.uint8, device=ids.device) if scratch_bytes else None),
    )
    return output


def _validate_metadata(topk_ids: torch.Tensor, *, block_size: int, num_experts: int) -> int:
    """Checks on the route ids and sizes before anything is allocated or
    launched; returns the fixed capacity.  Exception classes follow the
    reference (``deterministic_moe_align.py:136-160``): TypeError for a
    non-tensor or an element type other than int32 / int64, ValueError for
    the rest."""

    C.tensor("topk_ids", topk_ids, ndim=2, nonempty=True, dtype=(torch.int32, torch.int64), contiguous=True)
    C.positive_int("block_size", block_size)
    C.positive_int("num_experts", num_experts)
    if num_experts > 1024:
        raise ValueError(f"num_experts={num_experts}: the HIP alignment handles at most 1024 experts")
    capacity = max_padded_tokens(topk_ids.numel(), num_experts, block_size)
    if max(topk_ids.numel(), capacity, num_experts - 1) > torch.iinfo(torch.int32).max:
        raise ValueError("the alignment would not fit the int32 indices of the Marlin ABI")
    return capacity


def _validate_output(output: DeterministicMoEAlignment, *, topk_ids: torch.Tensor, block_size: int,
                     capacity: int) -> None:
    """The caller-owned output: three separate int32 buffers of the ABI sizes
    on the ids' device (reference ``:162-191``: TypeError for the wrong
    container or a non-tensor field, ValueError for every other mismatch)."""

    if not isinstance(output, DeterministicMoEAlignment):
        raise TypeError(f"output: expected DeterministicMoEAlignment, got {type(output).__name__}")
    sizes = {
        "sorted_token_ids": capacity,
        "expert_ids": -(-capacity // block_size),
        "num_tokens_post_padded": 1,
    }
    fields = {name: getattr(output, name) for name in sizes}
    for name, size in sizes.items():
        C.tensor(f"output.{name}", fields[name], shape=(size,), dtype=torch.int32, dtype_error=ValueError,
                 device=topk_ids.device, contiguous=True)
    C.distinct_storages(fields, what="alignment output")


__all__ = [
    "DeterministicMoEAlignment",
    "allocate_deterministic_moe_alignment",
    "deterministic_moe_align_block_size",
    "max_padded_tokens",
]
