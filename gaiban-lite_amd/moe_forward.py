"""Router (gate) entry points on the HIP kernels.

Drop-in for the gate half of ``runtime/dsv4_direct/moe_forward.py``:
``gate_forward_with_boundary`` / ``gate_forward`` / ``hash_gate_forward`` keep
their signatures, validation and outputs, generalised over the score function
of ``Gate.forward`` (``reference/inference/model.py:564-584``).  Logits come
from the HIP gate-GEMM kernel (bf16 MFMA, fp32 accumulation) and scores,
top-(k+1) selection, weights and margin from the HIP router kernel.
``route_from_logits`` is the same router for callers that already hold fp32
logits (the synthetic benchmark configurations).

The module's checkpoint dequantisers (``_decoded_e8m0``, ``dequant_mxfp4``,
``dequant_fp8_block``; reference ``moe_forward.py:115-176``) keep their
signatures and exception classes and run as HIP streaming kernels; they give
the dense fp32 weights a dense executor or a check needs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch

from . import contracts as C
from . import ops

FP4_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)


@dataclass(frozen=True)
class GateForwardTensors:
    routing_weights: torch.Tensor
    routing_ids: torch.Tensor
    margin: torch.Tensor
    selection_ids: torch.Tensor
    selection_scores: torch.Tensor


@dataclass(frozen=True)
class HashGateForwardTensors:
    routing_weights: torch.Tensor
    routing_ids: torch.Tensor
    selected_scores: torch.Tensor


def route_from_logits(
    logits: torch.Tensor,
    *,
    topk: int,
    score_func: str = "sigmoid",
    bias: torch.Tensor | None = None,
    route_scale: float = 1.0,
) -> GateForwardTensors:
    """Scores, selection, weights and margin from fp32 logits [T, E]."""

    if logits.ndim != 2:
        raise ValueError("logits must be [tokens, experts]")
    tokens, experts = logits.shape
    if not isinstance(topk, int) or isinstance(topk, bool) or not 0 < topk < experts:
        raise ValueError("topk must be a positive integer smaller than expert count")
    if topk > 16:
        raise ValueError("the HIP router supports topk <= 16")
    if not math.isfinite(route_scale) or route_scale <= 0:
        raise ValueError("route_scale must be finite and positive")
    logits = logits.float().contiguous()
    dev = logits.device
    ids = torch.empty((tokens, topk), dtype=torch.int32, device=dev)
    weights = torch.empty((tokens, topk), dtype=torch.float32, device=dev)
    margin = torch.empty((tokens,), dtype=torch.float32, device=dev)
    sel_ids = torch.empty((tokens, topk + 1), dtype=torch.int32, device=dev)
    sel_scores = torch.empty((tokens, topk + 1), dtype=torch.float32, device=dev)
    ops.route_topk_into(
        logits,
        None if bias is None else bias.float().contiguous(),
        topk=topk,
        score_func=score_func,
        route_scale=route_scale,
        ids=ids,
        weights=weights,
        margin=margin,
        selection_ids=sel_ids,
        selection_scores=sel_scores,
    )
    return GateForwardTensors(
        routing_weights=weights,
        routing_ids=ids,
        margin=margin,
        selection_ids=sel_ids.long(),
        selection_scores=sel_scores,
    )


def gate_logits(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp32 logits = x . W^T for bf16 x [T, H] and bf16 W [E, H]."""

    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x [T, H] and weight [E, H] must share H")
    xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
    wb = weight if weight.dtype == torch.bfloat16 else weight.to(torch.bfloat16)
    logits = torch.empty((x.shape[0], weight.shape[0]), dtype=torch.float32, device=x.device)
    ops.gate_logits_into(xb.contiguous(), wb.contiguous(), logits)
    return logits


def gate_forward_with_boundary(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    topk: int = 6,
    route_scale: float = 1.5,
    score_func: str = "sqrtsoftplus",
) -> GateForwardTensors:
    """Learned gate (``moe_forward.py:52-94``): bias shifts selection only;
    weights gather unbiased scores, are renormalised and times route_scale."""

    if x.ndim != 2 or weight.ndim != 2 or (bias is not None and bias.ndim != 1):
        raise ValueError("x/weight/bias must have ranks 2/2/1")
    experts, hidden = weight.shape
    if x.shape[1] != hidden:
        raise ValueError(f"x hidden size {x.shape[1]} != gate hidden size {hidden}")
    if bias is not None and bias.numel() != experts:
        raise ValueError(f"gate bias size {bias.numel()} != experts {experts}")
    if not isinstance(topk, int) or isinstance(topk, bool) or not 0 < topk < experts:
        raise ValueError("topk must be a positive integer smaller than expert count")
    if not math.isfinite(route_scale) or route_scale <= 0:
        raise ValueError("route_scale must be finite and positive")
    return route_from_logits(
        gate_logits(x, weight), topk=topk, score_func=score_func, bias=bias,
        route_scale=route_scale,
    )


def gate_forward(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    topk: int = 6,
    route_scale: float = 1.5,
    score_func: str = "sqrtsoftplus",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    result = gate_forward_with_boundary(
        x, weight, bias, topk=topk, route_scale=route_scale, score_func=score_func
    )
    return result.routing_weights, result.routing_ids, result.margin


def hash_gate_forward(
    x: torch.Tensor,
    weight: torch.Tensor,
    tid2eid: torch.Tensor,
    input_ids: torch.Tensor,
    *,
    route_scale: float = 1.5,
) -> HashGateForwardTensors:
    """Token-id router of layers 0-2 (``moe_forward.py:186-231``)."""

    x = C.tensor("x", x, ndim=2)
    weight = C.tensor("gate weight", weight, ndim=2)
    tid2eid = C.tensor("tid2eid", tid2eid, ndim=2)
    experts, hidden = weight.shape
    if x.shape[1] != hidden:
        raise ValueError(f"x has hidden size {x.shape[1]}, the gate {hidden}")
    C.tensor("input_ids", input_ids, shape=(x.shape[0],))
    C.tensor("input_ids", input_ids, dtype=torch.int64)
    C.tensor("tid2eid", tid2eid, dtype=torch.int64)
    if not 0 < tid2eid.shape[1] < experts:
        raise ValueError(f"tid2eid routes {tid2eid.shape[1]} experts per token; need 1 .. {experts - 1}")
    C.same_device("hash gate tensors", (x, weight, tid2eid, input_ids))
    C.finite_positive("route_scale", route_scale)
    logits = gate_logits(x, weight)
    topk = tid2eid.shape[1]
    ids = torch.empty((x.shape[0], topk), dtype=torch.int32, device=x.device)
    weights = torch.empty((x.shape[0], topk), dtype=torch.float32, device=x.device)
    selected = torch.empty((x.shape[0], topk), dtype=torch.float32, device=x.device)
    ops.route_hash_into(logits, tid2eid.contiguous(), input_ids.contiguous(),
                        route_scale=route_scale, ids=ids, weights=weights, selected_scores=selected)
    return HashGateForwardTensors(routing_weights=weights, routing_ids=ids, selected_scores=selected)


E8M0 = torch.float8_e8m0fnu


def _decoded_e8m0(scale: torch.Tensor) -> torch.Tensor:
    """A scale tensor as fp32 (``moe_forward.py:115-123``): E8M0 or uint8
    codes are decoded by the HIP kernel (2^(c - 127); byte 0 -> 2^-127,
    byte 255 -> NaN, as torch's E8M0 conversion); a floating tensor is taken
    as already decoded and only widened to fp32."""

    C.tensor("scale", scale)
    if scale.dtype in (torch.uint8, E8M0):
        if scale.device.type != "cuda":
            raise ValueError("scale: E8M0 codes are decoded on the GPU; got a CPU tensor")
        return ops.decode_e8m0(scale.contiguous().view(torch.uint8))
    if scale.is_floating_point():
        return scale.contiguous().float()
    raise TypeError(f"scale: expected E8M0 or uint8 codes or an already decoded float tensor, not {scale.dtype}")


def _on_gpu(name: str, t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{name}: the dequantiser runs on the GPU; got a {t.device.type} tensor")


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Checkpoint MXFP4 weight -> fp32 [rows, 2 * packed.shape[1]]
    (``moe_forward.py:126-155``): byte b of a row holds logical K 2b in its
    low nibble and 2b+1 in its high nibble (E2M1 codes, values
    ``FP4_VALUES``), one E8M0 (or decoded) scale per 32 K.  Computed by the
    HIP kernel as one fp32 product per weight, bit-identical to the table
    lookup times the repeated scale."""

    C.tensor("packed", packed, ndim=2)
    C.tensor("scale", scale, ndim=2)
    C.tensor("packed", packed, dtype=(torch.int8, torch.uint8))
    rows, logical_k = packed.shape[0], 2 * packed.shape[1]
    if logical_k % 32:
        raise ValueError(f"packed: logical K = {logical_k} is not a multiple of the 32-wide scale group")
    C.tensor("scale", scale, shape=(rows, logical_k // 32))
    _on_gpu("packed", packed)
    codes = packed.contiguous().view(torch.uint8)
    return ops.dequant_mxfp4(codes, _decoded_e8m0(scale))


def dequant_fp8_block(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """128 x 128 block-scaled weight -> fp32 (``moe_forward.py:158-176``):
    ``weight[r, c] * scale[r // 128, c // 128]`` with the scale E8M0 codes or
    already decoded; rows and columns need not be multiples of 128.  The
    weight may be FP8 E4M3FN (the checkpoint's), bf16, fp16 or fp32."""

    C.tensor("weight", weight, ndim=2)
    C.tensor("scale", scale, ndim=2)
    rows, cols = weight.shape
    C.tensor("scale", scale, shape=(-(-rows // 128), -(-cols // 128)))
    C.tensor("weight", weight, dtype=tuple(ops.DTYPE_CODES))
    _on_gpu("weight", weight)
    return ops.dequant_fp8_block(weight, _decoded_e8m0(scale))


def error_metrics(observed: torch.Tensor, reference: torch.Tensor) -> dict[str, Any]:
    """JSON-safe max-absolute and relative-RMS error (``moe_forward.py:234-268``)."""

    if observed.shape != reference.shape:
        raise ValueError(
            f"observed shape {tuple(observed.shape)} != reference shape {tuple(reference.shape)}"
        )
    if observed.numel() == 0:
        raise ValueError("cannot compare empty tensors")
    o = observed.detach().float()
    r = reference.detach().float()
    if not bool(torch.isfinite(o).all().item() and torch.isfinite(r).all().item()):
        return {"finite": False, "max_abs": None, "rms_rel": None, "reference_rms": None}
    d = o - r
    ref_rms = r.square().mean().sqrt().item()
    return {
        "finite": True,
        "max_abs": float(d.abs().max().item()),
        "rms_rel": float(d.square().mean().sqrt().item() / max(ref_rms, torch.finfo(torch.float32).eps)),
        "reference_rms": float(ref_rms),
    }


__all__ = [
    "E8M0",
    "FP4_VALUES",
    "GateForwardTensors",
    "HashGateForwardTensors",
    "dequant_fp8_block",
    "dequant_mxfp4",
    "error_metrics",
    "gate_forward",
    "gate_forward_with_boundary",
    "gate_logits",
    "hash_gate_forward",
    "route_from_logits",
]
