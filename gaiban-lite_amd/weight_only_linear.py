"""W8A16 weight-only linear with the plan / caller-owned-storage interface of
``experiments/C1F-integrated-block/weight_only_linear.py``.

Kept from the reference: ``GemmPlan`` (m, n, k, split_k) freezing one launch
geometry with its caller-owned fp32 split-K workspace ``[split_k, M, N]``
(``:71-135``), ``make_gemm_plan`` (``:181-221``), the tensor validation raising
``TypeError`` / ``ValueError`` before any launch (``:334-432``),
``validate_non_alias_tensors`` (``:434-476``), and the hot wrapper
``w8a16_gemm_into(activation, weight, weight_scale, out, workspace, *, plan)``
(``:794-823``) that allocates nothing and never synchronises.

Two weight formats, each repacked once into the tiled layout of
``dsv4moe_pack_int8``:
  * int8 symmetric per output channel with a bf16 scale per row
    (``prepare_int8_weight``, ``w8a16_gemm_into``; the BASELINE format);
  * the reference checkpoint's FP8 E4M3 weights with one E8M0 scale per
    128 x 128 block (``prepare_fp8_block_weight``, ``w8a16_fp8_gemm_into``;
    E8M0 decode and the reserved-byte preflight of ``:488-513``).
The automatic split-K policy is the HIP library's
(``dsv4moe_w8a16_split_k``, sized for its 128/256-row workgroup tiles and
256 CUs) rather than ``_automatic_split_k`` (``:168-179``), which is tuned for
32x64 Triton tiles; split_k may also be 16.  The kernels are in
``csrc/linear.hip``.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass
from typing import Final

import torch

from . import ops

ACTIVATION_DTYPE: Final = torch.bfloat16
WEIGHT_DTYPE: Final = torch.int8
SCALE_DTYPE: Final = torch.bfloat16
OUTPUT_DTYPE: Final = torch.bfloat16
WORKSPACE_DTYPE: Final = torch.float32
BLOCK_K: Final = 128
SUPPORTED_SPLIT_K: Final = (1, 2, 4, 8, 16)

LAYOUT_CONTRACT: Final = {
    "activation": "row_major_bf16[M,K]",
    "weight": "tiled_int8[N*K] (16 rows x 64 K per 1 KiB tile)",
    "weight_scale": "bf16[N]",
    "output": "row_major_bf16[M,N]",
    "split_k_workspace": "row_major_fp32[split_k,M,N]",
    "activation_quantization": None,
    "materialized_bf16_weight": None,
}


@dataclass(frozen=True)
class GemmPlan:
    """Static launch and caller-owned storage contract."""

    m: int
    n: int
    k: int
    split_k: int

    @property
    def activation_shape(self) -> tuple[int, int]:
        return (self.m, self.k)

    @property
    def weight_shape(self) -> tuple[int]:
        return (self.n * self.k,)

    @property
    def weight_scale_shape(self) -> tuple[int]:
        return (self.n,)

    @property
    def output_shape(self) -> tuple[int, int]:
        return (self.m, self.n)

    @property
    def workspace_shape(self) -> tuple[int, ...]:
        return (0,) if self.split_k == 1 else (self.split_k, self.m, self.n)

    @property
    def workspace_elements(self) -> int:
        return 0 if self.split_k == 1 else self.split_k * self.m * self.n

    @property
    def workspace_bytes(self) -> int:
        return self.workspace_elements * 4

    @property
    def dispatch(self) -> str:
        return "full_k" if self.split_k == 1 else "split_k_reduce"


def _positive_dimension(name: str, value: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value!r}")
    return value


def make_gemm_plan(m: int, n: int, k: int, *, split_k: int | None = None) -> GemmPlan:
    """Freeze one geometry (``weight_only_linear.py:181-221``)."""

    m = _positive_dimension("m", m)
    n = _positive_dimension("n", n)
    k = _positive_dimension("k", k)
    if k % BLOCK_K:
        raise ValueError(f"k must be divisible by {BLOCK_K}, got {k}")
    if n % 16:
        raise ValueError(f"n must be divisible by 16, got {n}")
    selected = ops.w8a16_split_k(m, n, k) if split_k is None else split_k
    if isinstance(selected, bool) or not isinstance(selected, int) or selected not in SUPPORTED_SPLIT_K:
        raise ValueError(f"split_k must be one of {SUPPORTED_SPLIT_K}, got {selected!r}")
    if selected > k // BLOCK_K:
        raise ValueError(f"split_k={selected} exceeds K-block count {k // BLOCK_K}")
    return GemmPlan(m=m, n=n, k=k, split_k=selected)


def allocate_workspace(plan: GemmPlan, device) -> torch.Tensor:
    return torch.empty(plan.workspace_shape, dtype=WORKSPACE_DTYPE, device=device)


@dataclass(frozen=True)
class PreparedInt8Weight:
    """Tiled int8 weight (uint8 [N*K]) and its bf16 per-channel scale [N]."""

    packed: torch.Tensor
    scale: torch.Tensor
    n: int
    k: int


def prepare_int8_weight(weight: torch.Tensor, scale: torch.Tensor) -> PreparedInt8Weight:
    """Load-time repack of a row-major int8 [N, K] weight (device tensors)."""

    if not isinstance(weight, torch.Tensor) or not isinstance(scale, torch.Tensor):
        raise TypeError("weight and scale must be tensors")
    if weight.dtype != WEIGHT_DTYPE or weight.ndim != 2:
        raise TypeError("weight must be int8 [N, K]")
    n, k = weight.shape
    if scale.dtype != SCALE_DTYPE or tuple(scale.shape) != (n,):
        raise TypeError(f"scale must be bf16 [{n}]")
    if weight.device != scale.device:
        raise ValueError("weight and scale must share a device")
    packed = ops.pack_int8(weight.contiguous())
    return PreparedInt8Weight(packed=packed, scale=scale.contiguous(), n=n, k=k)


@dataclass(frozen=True)
class PreparedFP8BlockWeight:
    """Tiled FP8 E4M3 weight (uint8 [N*K]) and its E8M0 block scales
    (uint8 [ceil(N/128), K/128])."""

    packed: torch.Tensor
    scale: torch.Tensor
    n: int
    k: int


def validate_e8m0_scale_values(name: str, scale: torch.Tensor) -> None:
    """Cold preflight rejecting the reserved E8M0 byte 255 (``:488-500``);
    synchronises, so it belongs to load time."""

    codes = scale.view(torch.uint8) if scale.dtype == torch.float8_e8m0fnu else scale
    if codes.dtype != torch.uint8:
        raise TypeError(f"{name} must be uint8 or float8_e8m0fnu, got {scale.dtype}")
    if bool((codes == 255).any().item()):
        raise ValueError(f"{name} contains reserved E8M0 byte 255")


def prepare_fp8_block_weight(weight: torch.Tensor, scale: torch.Tensor) -> PreparedFP8BlockWeight:
    """Load-time repack of a row-major FP8 E4M3 [N, K] weight (float8_e4m3fn
    or its uint8 codes) with E8M0 scales [ceil(N/128), K/128] (float8_e8m0fnu
    or uint8 codes), the checkpoint's block-scaled format."""

    if not isinstance(weight, torch.Tensor) or not isinstance(scale, torch.Tensor):
        raise TypeError("weight and scale must be tensors")
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8) or weight.ndim != 2:
        raise TypeError("weight must be float8_e4m3fn (or its uint8 codes) [N, K]")
    n, k = weight.shape
    if k % BLOCK_K:
        raise ValueError(f"K={k} must be a multiple of {BLOCK_K}")
    if scale.dtype not in (torch.float8_e8m0fnu, torch.uint8) or tuple(scale.shape) != ((n + 127) // 128, k // 128):
        raise TypeError(f"scale must be float8_e8m0fnu (or uint8 codes) [{(n + 127) // 128}, {k // 128}]")
    if weight.device != scale.device:
        raise ValueError("weight and scale must share a device")
    validate_e8m0_scale_values("scale", scale)
    codes = scale.view(torch.uint8) if scale.dtype == torch.float8_e8m0fnu else scale
    packed = ops.pack_fp8(weight.contiguous())
    return PreparedFP8BlockWeight(packed=packed, scale=codes.contiguous(), n=n, k=k)


def _check_tensor(name, tensor, *, shape, dtype, device) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tuple(tensor.shape) != tuple(shape):
        raise ValueError(f"{name} shape must be {tuple(shape)}, got {tuple(tensor.shape)}")
    if tensor.dtype != dtype:
        raise TypeError(f"{name} dtype must be {dtype}, got {tensor.dtype}")
    if tensor.device != device:
        raise ValueError(f"{name} must be on {device}, got {tensor.device}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def validate_w8a16_tensors(activation, weight, weight_scale, out, workspace, *, plan: GemmPlan) -> torch.device:
    """Validate metadata without launching or synchronising."""

    if not isinstance(plan, GemmPlan):
        raise TypeError("plan must be GemmPlan")
    if not isinstance(activation, torch.Tensor):
        raise TypeError("activation must be a tensor")
    device = activation.device
    _check_tensor("activation", activation, shape=plan.activation_shape, dtype=ACTIVATION_DTYPE, device=device)
    _check_tensor("weight", weight, shape=plan.weight_shape, dtype=torch.uint8, device=device)
    _check_tensor("weight_scale", weight_scale, shape=plan.weight_scale_shape, dtype=SCALE_DTYPE, device=device)
    _check_tensor("out", out, shape=plan.output_shape, dtype=OUTPUT_DTYPE, device=device)
    _check_tensor("workspace", workspace, shape=plan.workspace_shape, dtype=WORKSPACE_DTYPE, device=device)
    return device


def validate_non_alias_tensors(tensors: Mapping[str, torch.Tensor]) -> None:
    """Cold preflight: one device, contiguous, no overlapping storage spans
    (empty tensors, such as the split-1 workspace, cannot alias)."""

    if not isinstance(tensors, Mapping) or not tensors:
        raise ValueError("non-alias tensor mapping must be non-empty")
    device = None
    spans: list[tuple[str, int, int]] = []
    for name, tensor in tensors.items():
        if not isinstance(name, str) or not name:
            raise ValueError("non-alias tensor names must be non-empty strings")
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise ValueError(f"non-alias tensors must share one device: {name} is on {tensor.device}")
        if tensor.numel() == 0:
            continue
        start = int(tensor.data_ptr())
        stop = start + tensor.numel() * tensor.element_size()
        for other, a, b in spans:
            if start < b and a < stop:
                raise ValueError(f"linear tensor storage must not alias: {other} overlaps {name}")
        spans.append((name, start, stop))


def w8a16_gemm_into(activation: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                    out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """out = bf16(activation . (q * s)^T) into caller-owned storage; no
    allocation, no synchronisation (graph-capturable)."""

    validate_w8a16_tensors(activation, weight, weight_scale, out, workspace, plan=plan)
    if activation.device.type != "cuda":
        raise ValueError(f"linear tensors must be device tensors, got {activation.device}")
    ops.w8a16_linear_into(activation, weight, weight_scale, out,
                          workspace if plan.split_k > 1 else None, n=plan.n, split_k=plan.split_k)


def w8a16_fp8_gemm_into(activation: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                        out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """out = bf16(activation . bf16(q * 2^(e-127))^T) for FP8 E4M3 weights with
    E8M0 128 x 128 block scales (``prepare_fp8_block_weight``) into
    caller-owned storage; no allocation, no synchronisation."""

    if not isinstance(plan, GemmPlan):
        raise TypeError("plan must be GemmPlan")
    if not isinstance(activation, torch.Tensor):
        raise TypeError("activation must be a tensor")
    device = activation.device
    _check_tensor("activation", activation, shape=plan.activation_shape, dtype=ACTIVATION_DTYPE, device=device)
    _check_tensor("weight", weight, shape=plan.weight_shape, dtype=torch.uint8, device=device)
    _check_tensor("weight_scale", weight_scale, shape=((plan.n + 127) // 128, plan.k // BLOCK_K),
                  dtype=torch.uint8, device=device)
    _check_tensor("out", out, shape=plan.output_shape, dtype=OUTPUT_DTYPE, device=device)
    _check_tensor("workspace", workspace, shape=plan.workspace_shape, dtype=WORKSPACE_DTYPE, device=device)
    if device.type != "cuda":
        raise ValueError(f"linear tensors must be device tensors, got {device}")
    ops.w8a16_fp8_linear_into(activation, weight, weight_scale, out,
                              workspace if plan.split_k > 1 else None, n=plan.n, split_k=plan.split_k)


def w8a16_linear(activation: torch.Tensor, prepared, *, split_k: int | None = None) -> torch.Tensor:
    """Allocating convenience wrapper (cold paths and tests) for either
    prepared format."""

    m = activation.shape[0]
    plan = make_gemm_plan(m, prepared.n, prepared.k, split_k=split_k)
    out = torch.empty(plan.output_shape, dtype=OUTPUT_DTYPE, device=activation.device)
    ws = allocate_workspace(plan, activation.device)
    if isinstance(prepared, PreparedFP8BlockWeight):
        w8a16_fp8_gemm_into(activation, prepared.packed, prepared.scale, out, ws, plan=plan)
    else:
        w8a16_gemm_into(activation, prepared.packed, prepared.scale, out, ws, plan=plan)
    return out


__all__ = [
    "ACTIVATION_DTYPE",
    "BLOCK_K",
    "GemmPlan",
    "LAYOUT_CONTRACT",
    "OUTPUT_DTYPE",
    "PreparedFP8BlockWeight",
    "PreparedInt8Weight",
    "SUPPORTED_SPLIT_K",
    "WORKSPACE_DTYPE",
    "allocate_workspace",
    "make_gemm_plan",
    "prepare_fp8_block_weight",
    "prepare_int8_weight",
    "validate_e8m0_scale_values",
    "validate_non_alias_tensors",
    "validate_w8a16_tensors",
    "w8a16_fp8_gemm_into",
    "w8a16_gemm_into",
    "w8a16_linear",
]
