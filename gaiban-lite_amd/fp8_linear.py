"""Block-FP8 W8A8 dense linear on the HIP kernels.

Drop-in for ``runtime/dsv4_direct/fp8_linear.py``: the same constants, plan
dataclasses, validation and caller-owned storage (``activation_quant_into``,
``block_fp8_gemm_into``), computed by ``act_quant_block_fp8_kernel`` and
``w8a8_block_kernel`` (gfx950 block-scaled fp8 MFMA, both E8M0 block scales
applied inside the MFMA) instead of Triton.

Differences a caller sees:
* the weight is the ``PreparedFP8BlockWeight`` of
  ``weight_only_linear.prepare_fp8_block_weight`` (a load-time byte
  permutation of the checkpoint tensor into 1 KiB MFMA tiles).  A raw
  checkpoint ``float8_e4m3fn [N, K]`` tensor is accepted too and repacked on
  every call, which allocates;
* ``make_gemm_plan``'s automatic split follows this library's policy
  (``dsv4moe_block_fp8_split_k``: widen K while the grid is below 512
  workgroups), not the Triton tile count; explicit values are validated as
  in the reference, and the workspace shape follows the chosen split;
* N must be a multiple of 16 and K at most 32768.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Final

import torch

from . import ops
from .weight_only_linear import PreparedFP8BlockWeight, prepare_fp8_block_weight

SCHEMA: Final = "dsv4.e1b2g.block_fp8_primitives.v1"
FP8_DTYPE: Final = torch.float8_e4m3fn
E8M0_DTYPE: Final = torch.float8_e8m0fnu
OUTPUT_DTYPE: Final = torch.bfloat16
WEIGHT_BLOCK_N: Final = 128
BLOCK_K: Final = 128
FP8_MAX: Final = 448.0
MIN_ACTIVATION_AMAX: Final = 1.0e-4
SUPPORTED_SPLIT_K: Final = (1, 2, 4, 8)

LAYOUT_CONTRACT: Final = {
    "activation": "row_major[M,K]",
    "activation_quantized": "row_major[M,K]",
    "activation_scale": "row_major[M,K/128]",
    "weight": "checkpoint_row_major[N,K]",
    "weight_scale": "checkpoint_row_major[ceil(N/128),K/128]",
    "output": "row_major[M,N]",
    "split_k_workspace": "row_major[split_k,M,N]",
    "workspace_dtype": "torch.float32",
    "output_dtype": "torch.bfloat16",
    "grouped_wo_a_supported": False,
}


def _ceil_div(value: int, divisor: int) -> int:
    return (value + divisor - 1) // divisor


def _positive_dimension(name: str, value: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value!r}")
    return value


@dataclass(frozen=True)
class QuantizationPlan:
    """Activation block quantisation layout (``fp8_linear.py:53-71``)."""

    m: int
    k: int
    block_m: int = 16
    block_k: int = BLOCK_K

    @property
    def quantized_shape(self) -> tuple[int, int]:
        return (self.m, self.k)

    @property
    def scale_shape(self) -> tuple[int, int]:
        return (self.m, self.k // self.block_k)

    @property
    def grid(self) -> tuple[int, int]:
        return (_ceil_div(self.m, self.block_m), self.k // self.block_k)


@dataclass(frozen=True)
class GemmTuning:
    """The reference's Triton tile parameters (``:74-81``); validated and kept
    for plan identity, the HIP kernel picks its own tiles."""

    block_m: int = 32
    block_n: int = 64
    num_warps: int = 4
    num_stages: int = 3


DEFAULT_GEMM_TUNING: Final = GemmTuning()


@dataclass(frozen=True)
class GemmPlan:
    """Dispatch decision and caller-owned workspace contract (``:87-153``)."""

    m: int
    n: int
    k: int
    split_k: int
    tuning: GemmTuning = DEFAULT_GEMM_TUNING

    @property
    def activation_shape(self) -> tuple[int, int]:
        return (self.m, self.k)

    @property
    def activation_scale_shape(self) -> tuple[int, int]:
        return (self.m, self.k // BLOCK_K)

    @property
    def weight_shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def weight_scale_shape(self) -> tuple[int, int]:
        return (_ceil_div(self.n, WEIGHT_BLOCK_N), self.k // BLOCK_K)

    @property
    def output_shape(self) -> tuple[int, int]:
        return (self.m, self.n)

    @property
    def output_grid(self) -> tuple[int, int]:
        return (_ceil_div(self.m, self.tuning.block_m), _ceil_div(self.n, self.tuning.block_n))

    @property
    def gemm_grid(self) -> tuple[int, ...]:
        return self.output_grid if self.split_k == 1 else (*self.output_grid, self.split_k)

    @property
    def k_blocks_per_split(self) -> int:
        return _ceil_div(self.k // BLOCK_K, self.split_k)

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


def make_quantization_plan(m: int, k: int, *, block_m: int = 16) -> QuantizationPlan:
    """``make_quantization_plan`` (``:168-183``)."""

    m = _positive_dimension("m", m)
    k = _positive_dimension("k", k)
    block_m = _positive_dimension("block_m", block_m)
    if k % BLOCK_K:
        raise ValueError(f"k must be divisible by {BLOCK_K}, got {k}")
    if block_m not in (1, 2, 4, 8, 16, 32):
        raise ValueError(f"unsupported quantization block_m={block_m}")
    return QuantizationPlan(m=m, k=k, block_m=block_m)


def _validate_tuning(tuning: GemmTuning) -> None:
    if tuning.block_m not in (16, 32, 64):
        raise ValueError(f"unsupported GEMM block_m={tuning.block_m}")
    if tuning.block_n not in (32, 64, 128):
        raise ValueError(f"unsupported GEMM block_n={tuning.block_n}")
    if tuning.num_warps not in (4, 8):
        raise ValueError(f"unsupported GEMM num_warps={tuning.num_warps}")
    if tuning.num_stages not in (2, 3, 4):
        raise ValueError(f"unsupported GEMM num_stages={tuning.num_stages}")


def make_gemm_plan(m: int, n: int, k: int, *, split_k: int | None = None,
                   tuning: GemmTuning = DEFAULT_GEMM_TUNING) -> GemmPlan:
    """``make_gemm_plan`` (``:218-240``); the automatic split is this
    library's (``ops.block_fp8_split_k``)."""

    m = _positive_dimension("m", m)
    n = _positive_dimension("n", n)
    k = _positive_dimension("k", k)
    _validate_tuning(tuning)
    if k % BLOCK_K:
        raise ValueError(f"k must be divisible by {BLOCK_K}, got {k}")
    selected = ops.block_fp8_split_k(m, n, k) if split_k is None else split_k
    if isinstance(selected, bool) or selected not in SUPPORTED_SPLIT_K:
        raise ValueError(f"split_k must be one of {SUPPORTED_SPLIT_K}, got {selected!r}")
    if selected > k // BLOCK_K:
        raise ValueError(f"split_k={selected} exceeds K-block count {k // BLOCK_K}")
    return GemmPlan(m=m, n=n, k=k, split_k=selected, tuning=tuning)


def primitive_contract() -> dict[str, object]:
    """JSON-friendly identity (``:243-270``)."""

    return {
        "schema": SCHEMA,
        "block_k": BLOCK_K,
        "weight_block_n": WEIGHT_BLOCK_N,
        "fp8_dtype": str(FP8_DTYPE),
        "scale_dtypes": [str(E8M0_DTYPE)],
        "supported_split_k": list(SUPPORTED_SPLIT_K),
        "default_tuning": {
            "block_m": DEFAULT_GEMM_TUNING.block_m,
            "block_n": DEFAULT_GEMM_TUNING.block_n,
            "num_warps": DEFAULT_GEMM_TUNING.num_warps,
            "num_stages": DEFAULT_GEMM_TUNING.num_stages,
        },
        "layout": dict(LAYOUT_CONTRACT),
        "caller_preallocated": ["activation_quantized", "activation_scale", "output", "workspace"],
        "cuda_graph_friendly": True,
    }


def _check_tensor(name: str, tensor: torch.Tensor, *, shape: tuple[int, ...],
                  dtypes: tuple[torch.dtype, ...], device: torch.device) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tuple(tensor.shape) != shape:
        raise ValueError(f"{name} shape must be {shape}, got {tuple(tensor.shape)}")
    if tensor.dtype not in dtypes:
        expected = ", ".join(str(d) for d in dtypes)
        raise TypeError(f"{name} dtype must be one of ({expected}), got {tensor.dtype}")
    if tensor.device != device:
        raise ValueError(f"{name} must be on {device}, got {tensor.device}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _scale_codes(scale: torch.Tensor) -> torch.Tensor:
    if scale.dtype != E8M0_DTYPE:
        raise TypeError(f"scale must use {E8M0_DTYPE}, got {scale.dtype}")
    return scale.view(torch.uint8)


def validate_e8m0_scale_values(name: str, scale: torch.Tensor) -> None:
    """Reject the reserved E8M0 NaN byte once, outside captured paths (``:301-309``)."""

    if not isinstance(name, str) or not name:
        raise ValueError("scale preflight requires a non-empty name")
    if scale.dtype != E8M0_DTYPE:
        raise TypeError(f"{name} must use {E8M0_DTYPE}, got {scale.dtype}")
    if bool((scale.view(torch.uint8) == 255).any().item()):
        raise ValueError(f"{name} contains reserved E8M0 byte 255")


def activation_quant_into(x: torch.Tensor, quantized_out: torch.Tensor, scale_out: torch.Tensor, *,
                          plan: QuantizationPlan) -> None:
    """Quantise ``x`` into caller-owned FP8 and power-of-two scale buffers
    (``activation_quant_into``, ``:523-569``)."""

    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise ValueError("x must be a device tensor")
    _check_tensor("x", x, shape=plan.quantized_shape, dtypes=(torch.bfloat16, torch.float16, torch.float32),
                  device=x.device)
    _check_tensor("quantized_out", quantized_out, shape=plan.quantized_shape, dtypes=(FP8_DTYPE,), device=x.device)
    _check_tensor("scale_out", scale_out, shape=plan.scale_shape, dtypes=(E8M0_DTYPE,), device=x.device)
    ops.act_quant_block_fp8_into(x, quantized_out.view(torch.uint8), _scale_codes(scale_out))


def block_fp8_gemm_into(activation: torch.Tensor, activation_scale: torch.Tensor,
                        weight: PreparedFP8BlockWeight | torch.Tensor, weight_scale: torch.Tensor | None,
                        out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """Full-K or deterministic split-K block-FP8 GEMM into ``out``
    (``block_fp8_gemm_into``, ``:572-684``)."""

    if not isinstance(activation, torch.Tensor) or activation.device.type != "cuda":
        raise ValueError("activation must be a device tensor")
    device = activation.device
    _check_tensor("activation", activation, shape=plan.activation_shape, dtypes=(FP8_DTYPE,), device=device)
    _check_tensor("activation_scale", activation_scale, shape=plan.activation_scale_shape, dtypes=(E8M0_DTYPE,),
                  device=device)
    if isinstance(weight, PreparedFP8BlockWeight):
        if (weight.n, weight.k) != plan.weight_shape:
            raise ValueError(f"weight shape must be {plan.weight_shape}, got {(weight.n, weight.k)}")
        if weight_scale is not None:
            _check_tensor("weight_scale", weight_scale, shape=plan.weight_scale_shape, dtypes=(E8M0_DTYPE,),
                          device=device)
            if not torch.equal(_scale_codes(weight_scale), weight.scale):
                raise ValueError("weight_scale differs from the prepared weight's scales")
        prepared = weight
    else:
        _check_tensor("weight", weight, shape=plan.weight_shape, dtypes=(FP8_DTYPE,), device=device)
        _check_tensor("weight_scale", weight_scale, shape=plan.weight_scale_shape, dtypes=(E8M0_DTYPE,),
                      device=device)
        prepared = prepare_fp8_block_weight(weight, weight_scale)
    _check_tensor("out", out, shape=plan.output_shape, dtypes=(OUTPUT_DTYPE,), device=device)
    _check_tensor("workspace", workspace, shape=plan.workspace_shape, dtypes=(torch.float32,), device=device)
    ops.block_fp8_gemm_into(
        activation.view(torch.uint8), _scale_codes(activation_scale), prepared.packed, prepared.scale, out,
        workspace if plan.split_k > 1 else None, n=plan.n, split_k=plan.split_k,
    )


__all__ = [
    "BLOCK_K",
    "DEFAULT_GEMM_TUNING",
    "E8M0_DTYPE",
    "FP8_DTYPE",
    "GemmPlan",
    "GemmTuning",
    "LAYOUT_CONTRACT",
    "OUTPUT_DTYPE",
    "QuantizationPlan",
    "SCHEMA",
    "SUPPORTED_SPLIT_K",
    "WEIGHT_BLOCK_N",
    "activation_quant_into",
    "block_fp8_gemm_into",
    "make_gemm_plan",
    "make_quantization_plan",
    "primitive_contract",
    "validate_e8m0_scale_values",
]
