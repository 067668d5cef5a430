"""Torch restatement of the reference's dense MoE path.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: ``tests/`` use it as a
checker and ``bench.py`` times it as the CPU baseline.  The product path never
imports it.

The reference's correctness executor for the routed experts is
``DenseRoutedExecutor.__call__`` (``runtime/dsv4_direct/ops/dense_moe.py:289-354``):
sort the flat (token, slot) assignments by expert (stable), dequantise a chunk
of experts at a time, per expert gather its rows and run
``x @ w13^T -> fp32 clamp / SiLU * up -> h @ w2^T`` into an expert-major
scratch, multiply by the route weight in fp32 on the w2 output, undo the sort
with ``index_copy_`` and sum the top-k axis.  The shared expert is
``shared_bf16_partial`` (``moe_runtime.py:246-263``: separate w1 and w3
linears, fp32 clamp / SiLU, bf16 cast, w2 linear) and the two parts are added
with ``torch.add`` (``moe_runtime.py:1865-1873``).  The router is
``gate_forward_with_boundary`` (``moe_forward.py:52-94``) with the score
function of ``Gate.forward`` (``reference/inference/model.py:564-584``).

``dense_moe(..., dtype=torch.bfloat16)`` runs that op order in bf16 exactly as
the reference does (the CPU baseline).  ``dtype=torch.float32`` runs the same
structure with every tensor in fp32 and no intermediate rounding: the "fp32
accumulation of the same dequantized weights" the north star compares against
(with TF32 disabled on the GPU).

Weight formats: int4 two's complement with one bf16 scale per 128 K (low
nibble = even K), and MXFP4 (E2M1 codes, one E8M0 scale per 32 K;
``moe_forward.py:23-40,115-155``).  A clamp limit of 0 disables the clamp
(this build's convention; the reference always clamps, Flash uses 10).

Pinned by: ``tests/test_oracle_torch_path.py`` (bf16 mode against the numpy
mirror ``moe_bf16_mirror``: >= 99.9% of the outputs bit-identical, the rest
within 2^-8 of the largest output -- fp32 summation order differs -- while
dropping any single bf16 cast of the mirror falls below 90%; fp32 mode
against ``moe_fp32``; dequantisers bit-exact against the numpy ones) and the
GPU tests of the full layer (fp32 mode on the GPU against ``moe_fp32`` on
rows covering every alignment block).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

FP4_TABLE = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


INT4_TABLE = tuple(range(8)) + tuple(range(-8, 0))


def _byte_pair_table(values, device, dtype) -> torch.Tensor:
    """[256, 2] table: byte b -> (value of its low nibble, value of its high
    nibble), the structure of ``_byte_pair_table`` (``ops/dense_moe.py:41-50``)."""

    v = torch.tensor(values, dtype=torch.float32, device=device)
    b = torch.arange(256, device=device)
    return torch.stack((v[b & 0xF], v[b >> 4]), dim=-1).to(dtype)


def dequant_int4_g128(packed: torch.Tensor, scale: torch.Tensor, *, dtype=torch.float32) -> torch.Tensor:
    """``W[n, k] = q[n, k] * s[n, k // 128]`` with q the signed nibble (low
    nibble = even k), by byte-pair table lookup as ``dequant_mxfp4_bf16``
    (``ops/dense_moe.py:53-68``) does.  fp32: exact; bf16: the product rounded
    once to bf16."""

    pairs = _byte_pair_table(INT4_TABLE, packed.device, dtype)[packed.long()]
    return pairs.flatten(-2) * scale.to(dtype).repeat_interleave(128, dim=-1)


def decode_e8m0(codes: torch.Tensor) -> torch.Tensor:
    """E8M0 byte -> fp32 power of two (byte 0 -> 2^-127; 255 reserved):
    ``weight_only_linear.py:503-513``.  Built from the bit pattern so the
    subnormal 2^-127 survives on any device."""

    c = codes.view(torch.uint8).to(torch.int32)
    if bool((c == 255).any()):
        raise ValueError("reserved E8M0 byte 255")
    bits = torch.where(c == 0, torch.full_like(c, 1 << 22), c << 23)
    return bits.view(torch.float32)


def dequant_mxfp4(packed: torch.Tensor, scale_codes: torch.Tensor, *, dtype=torch.float32) -> torch.Tensor:
    """E2M1 codes times the E8M0 group scale (32 K): ``dequant_mxfp4``
    (``moe_forward.py:126-155``), by table lookup as ``dequant_mxfp4_bf16``
    (exact in bf16)."""

    pairs = _byte_pair_table(FP4_TABLE, packed.device, dtype)[packed.long()]
    return pairs.flatten(-2) * decode_e8m0(scale_codes).to(dtype).repeat_interleave(32, dim=-1)


@dataclass
class StackedExperts:
    """Checkpoint-layout experts stacked over the expert axis (index E is the
    shared expert when present).  ``fmt`` is "int4_g128" (bf16 scales) or
    "mxfp4" (E8M0 scale bytes)."""

    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    fmt: str = "int4_g128"

    def dequant(self, which: str, lo: int, hi: int, dtype) -> torch.Tensor:
        w, s = (self.w13, self.s13) if which == "w13" else (self.w2, self.s2)
        fn = dequant_int4_g128 if self.fmt == "int4_g128" else dequant_mxfp4
        return fn(w[lo:hi], s[lo:hi], dtype=dtype)


def _clamped_swiglu(gate: torch.Tensor, up: torch.Tensor, limit: float) -> torch.Tensor:
    g = gate.float()
    u = up.float()
    if limit > 0:
        g = g.clamp(max=limit)
        u = u.clamp(min=-limit, max=limit)
    return F.silu(g) * u


def routed_experts(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts: StackedExperts, *,
                   num_experts: int, clamp_limit: float = 0.0, dtype=torch.bfloat16,
                   expert_chunk: int = 8) -> torch.Tensor:
    """``DenseRoutedExecutor.__call__`` (``ops/dense_moe.py:289-354``) in
    ``dtype``; returns the routed partial [T, H] in ``dtype``."""

    rows, topk = ids.shape
    hidden = x.shape[1]
    inter = experts.w13.shape[1] // 2
    xin = x.to(dtype)
    flat_ids = ids.reshape(-1)
    flat_w = weights.reshape(-1).float()
    order = torch.argsort(flat_ids.to(torch.int32), stable=True)
    sorted_rows = torch.div(order, topk, rounding_mode="floor")
    counts = torch.bincount(flat_ids.long(), minlength=num_experts)
    bounds = [0] + torch.cumsum(counts, 0).tolist()
    scratch = torch.empty((rows * topk, hidden), dtype=dtype, device=x.device)
    for c0 in range(0, num_experts, expert_chunk):
        c1 = min(c0 + expert_chunk, num_experts)
        if bounds[c1] == bounds[c0]:
            continue
        w13 = experts.dequant("w13", c0, c1, dtype)
        w2 = experts.dequant("w2", c0, c1, dtype)
        for e in range(c0, c1):
            b, s = bounds[e], bounds[e + 1]
            if b == s:
                continue
            act = xin.index_select(0, sorted_rows[b:s])
            proj = act @ w13[e - c0].t()
            h = _clamped_swiglu(proj[:, :inter], proj[:, inter:], clamp_limit).to(dtype)
            scratch[b:s] = h @ w2[e - c0].t()
        del w13, w2
    weighted = scratch.float() * flat_w.index_select(0, order).unsqueeze(1)
    restored = torch.empty_like(weighted)
    restored.index_copy_(0, order, weighted)
    return restored.view(rows, topk, hidden).sum(dim=1).to(dtype)


def shared_partial(x: torch.Tensor, experts: StackedExperts, index: int, *, clamp_limit: float = 0.0,
                   dtype=torch.bfloat16) -> torch.Tensor:
    """``shared_bf16_partial`` (``moe_runtime.py:246-263``) in ``dtype``."""

    w13 = experts.dequant("w13", index, index + 1, dtype)[0]
    w2 = experts.dequant("w2", index, index + 1, dtype)[0]
    inter = w13.shape[0] // 2
    xin = x.to(dtype)
    act = _clamped_swiglu(F.linear(xin, w13[:inter]), F.linear(xin, w13[inter:]), clamp_limit).to(dtype)
    return F.linear(act, w2)


def dense_moe(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts: StackedExperts, *,
              num_experts: int, shared_index: int | None = None, clamp_limit: float = 0.0,
              dtype=torch.bfloat16, expert_chunk: int = 8) -> torch.Tensor:
    """Routed partial, shared partial and ``torch.add`` (``moe_runtime.py:1873``);
    fp32 mode sums in fp32 and returns fp32."""

    ctx = _highest_precision() if dtype == torch.float32 else _nullcontext()
    with ctx:
        routed = routed_experts(x, ids, weights, experts, num_experts=num_experts, clamp_limit=clamp_limit,
                                dtype=dtype, expert_chunk=expert_chunk)
        if shared_index is None:
            return routed
        shared = shared_partial(x, experts, shared_index, clamp_limit=clamp_limit, dtype=dtype)
        return torch.add(routed, shared)


class _nullcontext:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


class _highest_precision:
    """fp32 matmuls without TF32 / reduced-precision shortcuts."""

    def __enter__(self):
        self._tf32 = torch.backends.cuda.matmul.allow_tf32
        self._prec = torch.get_float32_matmul_precision()
        torch.backends.cuda.matmul.allow_tf32 = False
        torch.set_float32_matmul_precision("highest")
        return None

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.allow_tf32 = self._tf32
        torch.set_float32_matmul_precision(self._prec)
        return False


def gate_route(logits: torch.Tensor, *, topk: int, score_func: str = "sigmoid", bias: torch.Tensor | None = None,
               route_scale: float = 1.0):
    """``gate_forward_with_boundary`` (``moe_forward.py:80-87``) on fp32
    logits with the score function of ``Gate.forward`` (``model.py:565-571``):
    returns (ids int32 [T, k], weights fp32 [T, k], margin fp32 [T])."""

    lf = logits.float()
    if score_func == "sigmoid":
        scores = lf.sigmoid()
    elif score_func == "softmax":
        scores = lf.softmax(dim=-1)
    elif score_func == "sqrtsoftplus":
        scores = F.softplus(lf).sqrt()
    else:
        raise ValueError(f"unknown score function {score_func!r}")
    sel = scores if bias is None else scores + bias.float()
    values, picked = sel.topk(topk + 1, dim=-1)
    ids = picked[:, :topk]
    margin = values[:, topk - 1] - values[:, topk]
    w = scores.gather(1, ids)
    if score_func != "softmax":
        w = w / w.sum(dim=-1, keepdim=True)
    w = w * float(route_scale)
    return ids.to(torch.int32), w.float(), margin.float()


__all__ = [
    "FP4_TABLE",
    "StackedExperts",
    "decode_e8m0",
    "dense_moe",
    "dequant_int4_g128",
    "dequant_mxfp4",
    "gate_route",
    "routed_experts",
    "shared_partial",
]
