"""Block-FP8 W8A8 dense linear with the interface of
``runtime/dsv4_direct/fp8_linear.py``.

The reference quantises activations per row and 128-K block to E4M3 with a
power-of-two E8M0 scale (``activation_quant_into``, ``:523-569``) and runs
the GEMM over the checkpoint's E4M3 weight [N, K] with its E8M0 128 x 128
block scales, applying both scales per K block in fp32, with optional
deterministic split-K (``block_fp8_gemm_into``, ``:572-684``).  Here both
steps are HIP kernels: ``act_quant_block_fp8_kernel`` and the GEMM on
gfx950's block-scaled fp8 MFMA, which multiplies the two E8M0 scales into
each 128-K block product itself.

Kept: the module constants, ``QuantizationPlan`` / ``GemmPlan`` /
``GemmTuning`` with their fields, the two ``*_into`` entry points with
caller-owned storage, ``primitive_contract`` and
``validate_e8m0_scale_values``, and the exception classes of every check.
This build's own: the split policy (``dsv4moe_block_fp8_split_k``), the
kernels, and one extension -- ``block_fp8_gemm_into`` also takes a
``PreparedFP8BlockWeight`` (the weight repacked into MFMA tiles at load time)
in place of the raw weight, with ``weight_scale`` None; the output bits are
the same.  N must be a multiple of 16 and K at most 32768.
"""

from __future__ import annotations

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
from .weight_only_linear import PreparedFP8BlockWeight

SCHEMA: Final = "dsv4.e1b2g.block_fp8_primitives.v1"
FP8_DTYPE: Final = torch.float8_e4m3fn
E8M0_DTYPE: Final = torch.float8_e8m0fnu
OUTPUT_DTYPE: Final = torch.bfloat16
FP8_MAX: Final = 448.0
MIN_ACTIVATION_AMAX: Final = 1.0e-4
ACTIVATION_DTYPES: Final = (torch.bfloat16, torch.float16, torch.float32)
QUANT_BLOCK_M_CHOICES: Final = (1, 2, 4, 8, 16, 32)

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


@dataclass(frozen=True)
class QuantizationPlan:
    """Shapes of one activation quantisation (reference ``:53-71``): the
    quantised copy [M, K], one E8M0 scale per row and K block [M, K/128],
    and the reference's launch grid for ``block_m`` rows per program."""

    m: int
    k: int
    block_m: int = 16
    block_k: int = BLOCK_K

    quantized_shape = property(lambda self: (self.m, self.k))
    scale_shape = property(lambda self: (self.m, self.k // self.block_k))
    grid = property(lambda self: (-(-self.m // self.block_m), self.k // self.block_k))


def make_quantization_plan(m: int, k: int, *, block_m: int = 16) -> QuantizationPlan:
    """Validated quantisation plan (reference ``:166-181``); ValueError for
    any bad dimension."""

    m, k, block_m = (C.positive_int(name, v) for name, v in (("m", m), ("k", k), ("block_m", block_m)))
    if k % BLOCK_K:
        raise ValueError(f"k={k} is not a multiple of {BLOCK_K}")
    if block_m not in QUANT_BLOCK_M_CHOICES:
        raise ValueError(f"block_m={block_m} is not one of {QUANT_BLOCK_M_CHOICES}")
    return QuantizationPlan(m=m, k=k, block_m=block_m)


def make_gemm_plan(m: int, n: int, k: int, *, split_k: int | None = None,
                   tuning: GemmTuning = DEFAULT_GEMM_TUNING) -> GemmPlan:
    """One GEMM geometry (reference ``:207-234``); the automatic split is this
    library's policy for its kernel tiles."""

    return build_plan(m, n, k, split_k=split_k, tuning=tuning, policy=ops.block_fp8_split_k)


def primitive_contract() -> dict[str, object]:
    """A JSON-friendly description of the primitives (reference ``:237-261``)."""

    tuning = DEFAULT_GEMM_TUNING
    return {
        "schema": SCHEMA,
        "block_k": BLOCK_K,
        "weight_block_n": WEIGHT_BLOCK_N,
        "fp8_dtype": str(FP8_DTYPE),
        "scale_dtypes": [str(E8M0_DTYPE)],
        "supported_split_k": list(SUPPORTED_SPLIT_K),
        "default_tuning": {f: getattr(tuning, f) for f in ("block_m", "block_n", "num_warps", "num_stages")},
        "layout": dict(LAYOUT_CONTRACT),
        "caller_preallocated": ["activation_quantized", "activation_scale", "output", "workspace"],
        "cuda_graph_friendly": True,
    }


def _e8m0(name: str, value, shape, device) -> torch.Tensor:
    """A caller's E8M0 tensor as its uint8 byte view."""

    return C.tensor(name, value, shape=shape, dtype=E8M0_DTYPE, device=device, contiguous=True).view(torch.uint8)


def validate_e8m0_scale_values(name: str, scale: torch.Tensor) -> None:
    """Cold preflight against the reserved E8M0 byte 255 (reference
    ``:296-309``): ValueError for a bad name or the byte, TypeError unless the
    tensor is ``float8_e8m0fnu``.  Reads the device."""

    if not isinstance(name, str) or not name:
        raise ValueError("validate_e8m0_scale_values needs a non-empty name")
    C.tensor(name, scale, dtype=E8M0_DTYPE)
    C.no_reserved_e8m0(name, scale)


def _on_gpu(name: str, t) -> torch.device:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        where = t.device if isinstance(t, torch.Tensor) else type(t).__name__
        raise ValueError(f"{name} must be a device tensor, got {where}")
    return t.device


def activation_quant_into(x: torch.Tensor, quantized_out: torch.Tensor, scale_out: torch.Tensor, *,
                          plan: QuantizationPlan) -> None:
    """E4M3 codes and E8M0 scales of ``x`` into caller-owned tensors."""

    device = _on_gpu("x", x)
    C.tensor("x", x, shape=plan.quantized_shape, dtype=ACTIVATION_DTYPES, device=device, contiguous=True)
    q = C.tensor("quantized_out", quantized_out, shape=plan.quantized_shape, dtype=FP8_DTYPE, device=device,
                 contiguous=True)
    s = _e8m0("scale_out", scale_out, plan.scale_shape, device)
    ops.act_quant_block_fp8_into(x, q.view(torch.uint8), s)


def block_fp8_gemm_into(activation: torch.Tensor, activation_scale: torch.Tensor,
                        weight: torch.Tensor | PreparedFP8BlockWeight, weight_scale: torch.Tensor | None,
                        out: torch.Tensor, workspace: torch.Tensor, *, plan: GemmPlan) -> None:
    """Full-K or split-K block-FP8 GEMM into ``out``; the raw checkpoint
    weight is read as stored (no repack, no allocation)."""

    device = _on_gpu("activation", activation)
    a = C.tensor("activation", activation, shape=plan.activation_shape, dtype=FP8_DTYPE, device=device,
                 contiguous=True)
    a_scale = _e8m0("activation_scale", activation_scale, plan.activation_scale_shape, device)
    if isinstance(weight, PreparedFP8BlockWeight):
        if (weight.n, weight.k) != plan.weight_shape:
            raise ValueError(f"prepared weight is {(weight.n, weight.k)}, the plan needs {plan.weight_shape}")
        w_bytes, w_scale = weight.packed, weight.scale
        # A prepared weight carries its scales.  A weight_scale given beside it
        # must be the tensor it was prepared from (same storage and shape):
        # comparing values would read device memory back, a synchronisation
        # inside a call that may be captured.
        if weight_scale is not None:
            given = _e8m0("weight_scale", weight_scale, plan.weight_scale_shape, device)
            if given.data_ptr() != w_scale.data_ptr() or given.shape != w_scale.shape:
                raise ValueError("weight_scale is not the scale tensor the weight was prepared with; "
                                 "pass None with a prepared weight")
    else:
        w_bytes = C.tensor("weight", weight, shape=plan.weight_shape, dtype=FP8_DTYPE, device=device,
                           contiguous=True)
        w_scale = _e8m0("weight_scale", weight_scale, plan.weight_scale_shape, device)
    C.tensor("out", out, shape=plan.output_shape, dtype=OUTPUT_DTYPE, device=device, contiguous=True)
    C.tensor("workspace", workspace, shape=plan.workspace_shape, dtype=torch.float32, device=device,
             contiguous=True)
    ops.block_fp8_gemm_into(a.view(torch.uint8), a_scale, w_bytes, w_scale, out,
                            workspace if plan.split_k > 1 else None, n=plan.n, split_k=plan.split_k)


__all__ = [
    "ACTIVATION_DTYPES",
    "BLOCK_K",
    "DEFAULT_GEMM_TUNING",
    "E8M0_DTYPE",
    "FP8_DTYPE",
    "FP8_MAX",
    "GemmPlan",
    "GemmTuning",
    "LAYOUT_CONTRACT",
    "MIN_ACTIVATION_AMAX",
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
