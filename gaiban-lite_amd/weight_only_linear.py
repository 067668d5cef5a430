"""W8A16 weight-only linear with the interface of
``experiments/C1F-integrated-block/weight_only_linear.py``.

``w8a16_gemm_into(activation, weight, weight_scale, out, workspace, *, plan)``
(reference ``:794-823``) takes the checkpoint's tensors as stored: E4M3
``weight`` [N, K] (``float8_e4m3fn``) and E8M0 ``weight_scale``
[ceil(N/128), K/128] (``float8_e8m0fnu``), a bf16 activation [M, K], a bf16
output [M, N] and the fp32 split-K workspace of the plan; it validates
metadata only, allocates nothing and never synchronises, so it can be
captured in a graph.  The HIP kernel (``dsv4moe_w8a16_fp8_linear`` with the
row-major weight layout) converts each E4M3 code with its block's power of
two straight into the bf16 MFMA operand, which is the reference's
``bf16(q * 2^(e-127))`` exactly; fp32 accumulation, split-K partials summed
in split order, one bf16 rounding.

Variants of this build (no counterpart in the reference):
  * ``w8a16_prepared_gemm_into`` -- the same product over weights repacked
    once at load time into 1 KiB MFMA tiles (``prepare_fp8_block_weight`` /
    ``prepare_int8_weight``); the same output bits;
  * ``w8a16_int8_gemm_into`` -- the BASELINE format of this build's
    benchmark: int8 [N, K] weights with one bf16 scale per output channel
    (``weight_scale`` [N]), the scale applied once per output.

Plans (``GemmPlan``, ``make_gemm_plan``) are the shared plans of
``linear_plan.py``; the automatic split is this library's policy.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass
from typing import Final

import torch

from . import contracts as C
from . import ops
from .linear_plan import (
    BLOCK_K,
    DEFAULT_GEMM_TUNING,
    SUPPORTED_SPLIT_K,
    WEIGHT_BLOCK_N,
    GemmPlan,
    GemmTuning,
    build_plan,
)

SCHEMA: Final = "dsv4.e1b2q.weight_only_linear.v1"
ACTIVATION_DTYPE: Final = torch.bfloat16
FP8_DTYPE: Final = torch.float8_e4m3fn
E8M0_DTYPE: Final = torch.float8_e8m0fnu
OUTPUT_DTYPE: Final = torch.bfloat16
WORKSPACE_DTYPE: Final = torch.float32
INT8_WEIGHT_DTYPE: Final = torch.int8
INT8_SCALE_DTYPE: Final = torch.bfloat16
CANDIDATE_VARIANT: Final = "checkpoint_fp8_e8m0_weight_bf16_mma"

LAYOUT_CONTRACT: Final = {
    "activation": "row_major_bf16[M,K]",
    "candidate_weight": "checkpoint_row_major_e4m3[N,K]",
    "candidate_weight_scale": "checkpoint_row_major_e8m0[ceil(N/128),K/128]",
    "output": "row_major_bf16[M,N]",
    "split_k_workspace": "row_major_fp32[split_k,M,N]",
    "activation_quantization": None,
    "materialized_candidate_bf16_weight": None,
    "weight_sized_scratch": None,
}


def make_gemm_plan(m: int, n: int, k: int, *, split_k: int | None = None,
                   tuning: GemmTuning = DEFAULT_GEMM_TUNING) -> GemmPlan:
    """One geometry for every variant of this module (reference ``:182-221``)."""

    return build_plan(m, n, k, split_k=split_k, tuning=tuning, policy=ops.w8a16_split_k)


def allocate_workspace(plan: GemmPlan, device) -> torch.Tensor:
    """The plan's fp32 split-K workspace (cold path: allocates)."""

    return torch.empty(plan.workspace_shape, dtype=WORKSPACE_DTYPE, device=device)


def validate_e8m0_scale_values(name: str, scale: torch.Tensor) -> None:
    """Cold preflight against the reserved E8M0 byte 255 (reference
    ``:488-500``): ValueError for a bad name or the byte, TypeError for a
    non-tensor or another element type, ValueError for a strided tensor.
    Reads the device."""

    if not isinstance(name, str) or not name:
        raise ValueError("validate_e8m0_scale_values needs a non-empty name")
    C.tensor(name, scale, contiguous=True)
    C.no_reserved_e8m0(name, scale)


def decode_e8m0_scale_for_oracle(scale: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes -> fp32 powers of two for cold checks (reference
    ``:503-513``): byte 0 is 2^-127, byte b is 2^(b-127)."""

    validate_e8m0_scale_values("scale", scale)
    codes = C.e8m0_codes("scale", scale).to(torch.int32)
    exponent_field = torch.where(codes > 0, codes << 23, torch.full_like(codes, 1 << 22))
    return exponent_field.view(torch.float32)


def _check_io(activation, out, workspace, plan) -> torch.device:
    if not isinstance(plan, GemmPlan):
        raise TypeError(f"plan: expected GemmPlan, got {type(plan).__name__}")
    act = C.tensor("activation", activation, shape=plan.activation_shape, dtype=ACTIVATION_DTYPE,
                   contiguous=True)
    C.tensor("out", out, shape=plan.output_shape, dtype=OUTPUT_DTYPE, device=act.device, contiguous=True)
    C.tensor("workspace", workspace, shape=plan.workspace_shape, dtype=WORKSPACE_DTYPE, device=act.device,
             contiguous=True)
    return act.device


def validate_fp8_weight_only_tensors(activation, weight, weight_scale, out, workspace, *,
                                     plan: GemmPlan) -> torch.device:
    """Metadata of a ``w8a16_gemm_into`` call (reference ``:406-435``); no
    launch, no synchronisation."""

    device = _check_io(activation, out, workspace, plan)
    C.tensor("weight", weight, shape=plan.weight_shape, dtype=FP8_DTYPE, device=device, contiguous=True)
    C.tensor("weight_scale", weight_scale, shape=plan.weight_scale_shape, dtype=E8M0_DTYPE, device=device,
             contiguous=True)
    return device


def validate_non_alias_tensors(tensors: Mapping[str, torch.Tensor]) -> None:
    """Cold preflight (reference ``:437-477``): one device, contiguous,
    pairwise disjoint bytes (an empty tensor, such as the one-split
    workspace, holds none)."""

    C.byte_spans_disjoint(tensors, what="linear tensors")


def _launch_device(device: torch.device) -> None:
    if device.type != "cuda":
        raise ValueError(f"the linear runs on the GPU; tensors are on {device}")


def w8a16_gemm_into(activation: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                    out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """``out = bf16(activation . bf16(weight * 2^(e-127))^T)`` over the
    checkpoint's E4M3 weight and E8M0 block scales, into caller-owned
    storage (reference ``:794-823``)."""

    device = validate_fp8_weight_only_tensors(activation, weight, weight_scale, out, workspace, plan=plan)
    _launch_device(device)
    ops.w8a16_fp8_linear_into(activation, weight, weight_scale.view(torch.uint8), out,
                              workspace if plan.split_k > 1 else None, n=plan.n, split_k=plan.split_k)


fp8_weight_only_linear_into = w8a16_gemm_into


@dataclass(frozen=True)
class PreparedFP8BlockWeight:
    """E4M3 weight repacked into 1 KiB MFMA tiles (uint8 [N*K]) with its E8M0
    block scales as bytes (uint8 [ceil(N/128), K/128])."""

    packed: torch.Tensor
    scale: torch.Tensor
    n: int
    k: int


@dataclass(frozen=True)
class PreparedInt8Weight:
    """int8 weight repacked into 1 KiB MFMA tiles (uint8 [N*K]) with its bf16
    per-channel scale [N]."""

    packed: torch.Tensor
    scale: torch.Tensor
    n: int
    k: int


def prepare_fp8_block_weight(weight: torch.Tensor, scale: torch.Tensor) -> PreparedFP8BlockWeight:
    """Load-time repack of an E4M3 [N, K] weight (``float8_e4m3fn`` or its
    uint8 codes) and its E8M0 scales [ceil(N/128), K/128] (``float8_e8m0fnu``
    or uint8); rejects the reserved scale byte.  Allocates and synchronises."""

    C.tensor("weight", weight, ndim=2, dtype=(FP8_DTYPE, torch.uint8))
    n, k = weight.shape
    if k % BLOCK_K:
        raise ValueError(f"weight: K={k} is not a multiple of {BLOCK_K}")
    C.tensor("scale", scale, shape=(-(-n // WEIGHT_BLOCK_N), k // BLOCK_K), dtype=(E8M0_DTYPE, torch.uint8),
             shape_error=TypeError)
    C.same_device("weight and scale", (weight, scale))
    codes = C.e8m0_codes("scale", scale).contiguous()
    C.no_reserved_e8m0("scale", codes)
    return PreparedFP8BlockWeight(packed=ops.pack_fp8(weight.contiguous().view(torch.uint8)), scale=codes,
                                  n=n, k=k)


def prepare_int8_weight(weight: torch.Tensor, scale: torch.Tensor) -> PreparedInt8Weight:
    """Load-time repack of an int8 [N, K] weight with bf16 scales [N]."""

    C.tensor("weight", weight, ndim=2, dtype=INT8_WEIGHT_DTYPE, shape_error=TypeError)
    n, k = weight.shape
    C.tensor("scale", scale, shape=(n,), dtype=INT8_SCALE_DTYPE, shape_error=TypeError)
    C.same_device("weight and scale", (weight, scale))
    return PreparedInt8Weight(packed=ops.pack_int8(weight.contiguous()), scale=scale.contiguous(), n=n, k=k)


def w8a16_prepared_gemm_into(activation: torch.Tensor, prepared, out: torch.Tensor, workspace: torch.Tensor, *,
                             plan: GemmPlan) -> None:
    """``w8a16_gemm_into`` (FP8 blocks) or ``w8a16_int8_gemm_into`` (int8 per
    channel) over weights repacked at load time; same output bits."""

    device = _check_io(activation, out, workspace, plan)
    if not isinstance(prepared, (PreparedFP8BlockWeight, PreparedInt8Weight)):
        raise TypeError(f"prepared: expected a prepared weight, got {type(prepared).__name__}")
    if (prepared.n, prepared.k) != plan.weight_shape:
        raise ValueError(f"prepared weight is {(prepared.n, prepared.k)}, the plan needs {plan.weight_shape}")
    C.same_device("prepared weight and activation", (prepared.packed, prepared.scale, activation))
    _launch_device(device)
    ws = workspace if plan.split_k > 1 else None
    if isinstance(prepared, PreparedFP8BlockWeight):
        ops.w8a16_fp8_linear_into(activation, prepared.packed, prepared.scale, out, ws, n=plan.n,
                                  split_k=plan.split_k)
    else:
        ops.w8a16_linear_into(activation, prepared.packed, prepared.scale, out, ws, n=plan.n, split_k=plan.split_k)


def w8a16_int8_gemm_into(activation: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                         out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """``out = bf16(activation . (weight * scale[n])^T)``: int8 [N, K]
    weights as stored, one bf16 scale per output channel [N]."""

    device = _check_io(activation, out, workspace, plan)
    C.tensor("weight", weight, shape=plan.weight_shape, dtype=INT8_WEIGHT_DTYPE, device=device, contiguous=True)
    C.tensor("weight_scale", weight_scale, shape=(plan.n,), dtype=INT8_SCALE_DTYPE, device=device,
             contiguous=True)
    _launch_device(device)
    ops.w8a16_linear_into(activation, weight, weight_scale, out, workspace if plan.split_k > 1 else None,
                          n=plan.n, split_k=plan.split_k)


def w8a16_linear(activation: torch.Tensor, weight, weight_scale: torch.Tensor | None = None, *,
                 split_k: int | None = None) -> torch.Tensor:
    """Allocating convenience call for cold paths and tests: a prepared
    weight, or the checkpoint E4M3 weight with its E8M0 scales, or int8
    weights with bf16 per-channel scales."""

    m = activation.shape[0]
    n, k = (weight.n, weight.k) if weight_scale is None else tuple(weight.shape)
    plan = make_gemm_plan(m, n, k, split_k=split_k)
    out = torch.empty(plan.output_shape, dtype=OUTPUT_DTYPE, device=activation.device)
    ws = allocate_workspace(plan, activation.device)
    if weight_scale is None:
        w8a16_prepared_gemm_into(activation, weight, out, ws, plan=plan)
    elif weight.dtype == INT8_WEIGHT_DTYPE:
        w8a16_int8_gemm_into(activation, weight, weight_scale, out, ws, plan=plan)
    else:
        w8a16_gemm_into(activation, weight, weight_scale, out, ws, plan=plan)
    return out


__all__ = [
    "ACTIVATION_DTYPE",
    "BLOCK_K",
    "CANDIDATE_VARIANT",
    "DEFAULT_GEMM_TUNING",
    "E8M0_DTYPE",
    "FP8_DTYPE",
    "GemmPlan",
    "GemmTuning",
    "INT8_SCALE_DTYPE",
    "INT8_WEIGHT_DTYPE",
    "LAYOUT_CONTRACT",
    "OUTPUT_DTYPE",
    "PreparedFP8BlockWeight",
    "PreparedInt8Weight",
    "SCHEMA",
    "SUPPORTED_SPLIT_K",
    "WEIGHT_BLOCK_N",
    "WORKSPACE_DTYPE",
    "allocate_workspace",
    "decode_e8m0_scale_for_oracle",
    "fp8_weight_only_linear_into",
    "make_gemm_plan",
    "prepare_fp8_block_weight",
    "prepare_int8_weight",
    "validate_e8m0_scale_values",
    "validate_fp8_weight_only_tensors",
    "validate_non_alias_tensors",
    "w8a16_gemm_into",
    "w8a16_int8_gemm_into",
    "w8a16_linear",
    "w8a16_prepared_gemm_into",
]
