"""Deterministic fixed-capacity MoE alignment on the HIP align kernel.

Drop-in for ``runtime/dsv4_direct/deterministic_moe_align.py``: same dataclass,
same capacity rule, same validation, same output layout (the public
``moe_align_block_size`` ABI).  The layout is computed by one workgroup of the
HIP kernel ``align_kernel`` (ballot-ranked stable permutation), or for many
ids by the chunk-count and chunk-scatter kernels over a temporary scratch
tensor (in place of the reference's torch temporaries), with no host read of
route-dependent data.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops


@dataclass(frozen=True)
class DeterministicMoEAlignment:
    sorted_token_ids: torch.Tensor
    expert_ids: torch.Tensor
    num_tokens_post_padded: torch.Tensor


def max_padded_tokens(num_assignments: int, num_experts: int, block_size: int) -> int:
    """Fixed capacity (``deterministic_moe_align.py:17-32``)."""

    for name, value in (
        ("num_assignments", num_assignments),
        ("num_experts", num_experts),
        ("block_size", block_size),
    ):
        if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
            raise ValueError(f"{name} must be a positive integer")
    maximum = num_assignments + num_experts * (block_size - 1)
    if num_assignments < num_experts:
        maximum = min(num_assignments * block_size, maximum)
    return maximum


def allocate_deterministic_moe_alignment(
    topk_ids: torch.Tensor, *, block_size: int, num_experts: int
) -> DeterministicMoEAlignment:
    """Caller-owned output storage (``deterministic_moe_align.py:35-55``)."""

    _validate_metadata(topk_ids, block_size=block_size, num_experts=num_experts)
    maximum = max_padded_tokens(topk_ids.numel(), num_experts, block_size)
    return DeterministicMoEAlignment(
        sorted_token_ids=torch.empty(maximum, dtype=torch.int32, device=topk_ids.device),
        expert_ids=torch.empty(
            (maximum + block_size - 1) // block_size, dtype=torch.int32, device=topk_ids.device
        ),
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

    _validate_metadata(topk_ids, block_size=block_size, num_experts=num_experts)
    if topk_ids.device.type != "cuda":
        raise ValueError("deterministic_moe_align_block_size runs on the GPU; got a CPU tensor")
    if output is None:
        output = allocate_deterministic_moe_alignment(
            topk_ids, block_size=block_size, num_experts=num_experts
        )
    _validate_output(output, topk_ids=topk_ids, block_size=block_size, num_experts=num_experts)
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


def _validate_metadata(topk_ids: torch.Tensor, *, block_size: int, num_experts: int) -> None:
    if not isinstance(topk_ids, torch.Tensor):
        raise TypeError("topk_ids must be a tensor")
    if topk_ids.ndim != 2 or topk_ids.numel() == 0:
        raise ValueError("topk_ids must have non-empty shape [tokens, topk]")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_ids must use int32 or int64")
    if not topk_ids.is_contiguous():
        raise ValueError("topk_ids must be contiguous")
    for name, value in (("block_size", block_size), ("num_experts", num_experts)):
        if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
            raise ValueError(f"{name} must be a positive integer")
    if num_experts > 1024:
        raise ValueError("the HIP alignment supports at most 1024 experts")
    maximum = max_padded_tokens(topk_ids.numel(), num_experts, block_size)
    int32_max = torch.iinfo(torch.int32).max
    if topk_ids.numel() > int32_max or num_experts - 1 > int32_max or maximum > int32_max:
        raise ValueError("alignment metadata exceeds the int32 Marlin ABI")


def _validate_output(
    output: DeterministicMoEAlignment, *, topk_ids: torch.Tensor, block_size: int, num_experts: int
) -> None:
    if not isinstance(output, DeterministicMoEAlignment):
        raise TypeError("output must be DeterministicMoEAlignment")
    maximum = max_padded_tokens(topk_ids.numel(), num_experts, block_size)
    expected = (
        ("sorted_token_ids", output.sorted_token_ids, (maximum,)),
        ("expert_ids", output.expert_ids, ((maximum + block_size - 1) // block_size,)),
        ("num_tokens_post_padded", output.num_tokens_post_padded, (1,)),
    )
    pointers = set()
    for name, tensor, shape in expected:
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"output {name} must be a tensor")
        if tuple(tensor.shape) != shape or tensor.dtype != torch.int32:
            raise ValueError(f"output {name} shape/dtype differs from the ABI")
        if tensor.device != topk_ids.device or not tensor.is_contiguous():
            raise ValueError(f"output {name} device/layout differs from topk_ids")
        pointers.add(tensor.untyped_storage().data_ptr())
    if len(pointers) != len(expected):
        raise ValueError("alignment output tensors must not alias storage")


__all__ = [
    "DeterministicMoEAlignment",
    "allocate_deterministic_moe_alignment",
    "deterministic_moe_align_block_size",
    "max_padded_tokens",
]
