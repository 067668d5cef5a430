"""CPU restatement of gaiban-lite's DeepSeek-V4-Flash MoE hot path (numpy).

TEST INFRASTRUCTURE ONLY.  This module is the checker: ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` are the
only code allowed to import it.  The product path (the HIP extension behind
``include/dsv4moe.h``) never calls into it and fails loudly when the extension
is missing.

Every function cites the reference file:line it restates.  Paths are relative
to the gaiban-lite repository root.

What pins each function (checked in ``tests/test_oracle_*.py``):

* ``exp_f32`` / ``log_f32`` / ``log1p_f32`` / ``sigmoid_f32`` /
  ``sqrtsoftplus_f32`` / ``softmax_f32`` -- against float64 closed forms
  (<= 4 ULP) and special values (exp(0)=1, log(1)=0, sigmoid(0)=0.5, the
  softplus threshold x>20 -> x).
* ``route_topk`` -- brute force (``sorted`` with an explicit key) on small
  inputs, torch ``topk`` on rows without near-ties, the invariants of
  ``moe_runtime.py:463-475`` (row sum == route_scale within 8*eps*max(1,s)),
  margin >= 0, unique in-range ids.
* ``marlin_block_size_m`` / ``max_padded_tokens`` -- known answers
  (T=4,k=6,E=256 -> bs 8, cap 192; fixed B240 -> cap 3232, 404 blocks).
* ``moe_align`` -- the pure-list brute force of ``fixed_moe_align.py:424-456``
  (restated as ``moe_align_bruteforce``) on every small case, plus the layout
  invariants (multiset, ascending runs, padded multiples, -1 tail).
* ``dequant_int4_g128`` -- hand-packed known answers (nibble order, two's
  complement sign, group index) and a pack/unpack round trip.
* ``dequant_mxfp4`` / ``decode_e8m0`` -- the FP4 table KAT
  (``moe_forward.py:23-40``) and the E8M0 rule (``weight_only_linear.py:503-513``).
* ``moe_fp32`` -- a per-element scalar triple loop on tiny shapes, linearity in
  the route weights, and the reference op placement (weight on the w2 input).
* ``bf16_round`` / ``fp8_e4m3_round`` -- torch's own dtype conversions over
  every bf16 bit pattern / a dense sweep, and the exhaustive combine-add KAT
  of ``runtime/c2f_moe_combine_gate.py:54-84`` on a large sample.
* ``w8a16_linear_f32`` / ``automatic_split_k`` -- scalar loop on tiny shapes;
  split-K policy known answers from ``weight_only_linear.py:168-179``.
* ``act_quant_per_token_fp8`` -- torch's ``float8_e4m3fn`` cast of the same
  scaled, clamped values; ``moe_w4a8_f32`` -- a float64 pipeline built on that
  torch cast (quantised x, bf16 SwiGLU, quantised h, weight on the w2 output,
  shared expert) on tiny shapes.
* ``hash_route`` -- torch's own ``F.softplus(x).sqrt()`` -> ``index_select`` ->
  ``gather`` -> ``sum`` -> div -> ``* route_scale`` sequence
  (``moe_forward.py:218-223``) on seeded Flash-shape logits and random tables:
  ids equal, weights within 8 ulp (``tests/test_oracle_metrics.py``).
* ``error_metrics`` / ``rel_fro`` -- hand-computed known answers (an
  asymmetric pair that fixes which argument is the reference, the eps floor
  of the denominator, the non-finite, shape-mismatch and empty cases) and
  scale invariance (``tests/test_oracle_metrics.py``).
* ``running_sum_amplification`` / ``needs_exact_scaling`` -- hand-computed
  rows (a 2^100 group before a 2^-100 group, equal scales, a descending
  ramp) and the fp32 overflow they predict in a running-sum restatement
  (``tests/test_oracle_numerics.py``).
* ``moe_w4a8_mxfp4_f32`` -- the same float64 pipeline over torch's
  ``float8_e4m3fn`` cast and ``torch_path.dequant_mxfp4`` (itself bit-exact
  with the reference's dequantiser), with E8M0 scales spread over 2^-30 ..
  2^10 per 32-K group (``tests/test_oracle_ffn.py``).
* ``swiglu_f32`` -- torch's ``clamp`` / ``F.silu`` / multiply in
  ``Expert.forward``'s order, with planted clamp mistakes that fail
  (``tests/test_oracle_ffn.py``).
* ``route_scores`` -- through ``route_topk``'s brute force and the float64
  score closed forms (``tests/test_oracle_route_align.py``).
* ``fp8_e4m3_encode`` / ``fp8_e4m3_decode`` -- every code round trips and
  decodes as torch's ``float8_e4m3fn`` (``tests/test_oracle_numerics.py``).
* ``dequant_fp8_block`` -- torch's ``float8_e4m3fn`` times its
  ``float8_e8m0fnu`` block scale, bit for bit, ragged last block included;
  ``w8a16_fp8_linear_f32`` -- a scalar loop over the bf16-rounded weights
  (``tests/test_oracle_ffn.py``).
* ``act_quant_block_fp8`` -- codes and exponents equal a torch statement of
  the reference's quantiser (``fp8_linear.py:168-251``) incl. zero blocks and
  3e38; ``block_fp8_gemm_f32`` -- a float64 matmul of the dequantised operands
  (``tests/test_oracle_block_fp8.py``).
* ``shared_fp8_bf16`` -- the reference's torch op sequence
  (``moe_runtime.py:238-263``) bit for bit on dyadic operands
  (``tests/test_oracle_ffn.py``).
* ``moe_bf16_mirror`` -- against a torch restatement of the reference's bf16
  op order (torch's own bf16 matmuls, fp32 clamp / SiLU and casts): at least
  99.9% of the outputs bit-identical, the rest within 2^-8 of the largest
  output; removing any one of its bf16 rounding points drops agreement below
  90% (``tests/test_oracle_torch_path.py``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

F32 = np.float32

__all__ = [
    "BF16_CASTS",
    "FP4_VALUES",
    "SCORE_SIGMOID",
    "SCORE_SOFTMAX",
    "SCORE_SQRTSOFTPLUS",
    "AlignResult",
    "ExpertSource",
    "MXFP4ExpertSource",
    "RouteResult",
    "act_quant_block_fp8",
    "act_quant_per_token_fp8",
    "block_fp8_gemm_f32",
    "automatic_split_k",
    "bf16_bits_to_f32",
    "bf16_round",
    "bf16_to_bits",
    "decode_e8m0",
    "dequant_int4_g128",
    "dequant_mxfp4",
    "error_metrics",
    "exp_f32",
    "dequant_fp8_block",
    "fp8_e4m3_decode",
    "fp8_e4m3_encode",
    "fp8_e4m3_round",
    "hash_route",
    "log1p_f32",
    "log_f32",
    "marlin_block_size_m",
    "max_padded_tokens",
    "moe_align",
    "moe_align_bruteforce",
    "moe_bf16_mirror",
    "moe_fp32",
    "moe_w4a8_f32",
    "moe_w4a8_mxfp4_f32",
    "needs_exact_scaling",
    "running_sum_amplification",
    "pack_int4_rows",
    "rel_fro",
    "route_scores",
    "route_topk",
    "sigmoid_f32",
    "softmax_f32",
    "swiglu_f32",
    "sqrtsoftplus_f32",
    "unpack_int4_rows",
    "shared_fp8_bf16",
    "w8a16_fp8_linear_f32",
    "w8a16_linear_f32",
]

SCORE_SIGMOID = 0
SCORE_SOFTMAX = 1
SCORE_SQRTSOFTPLUS = 2

# ---------------------------------------------------------------------------
# bf16 / fp8 rounding (IEEE round-to-nearest-even)
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), kept as float32.

    Restates torch's ``Tensor.to(torch.bfloat16)``; used wherever the reference
    casts to bf16 (``ops/dense_moe.py:345``, ``moe_runtime.py:262,1873``).
    """

    a = np.ascontiguousarray(np.asarray(x, dtype=F32))
    bits = a.view(np.uint32)
    rounded = (bits + (np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1)))) & np.uint32(
        0xFFFF0000
    )
    nan = np.isnan(a)
    if nan.any():
        rounded = np.where(nan, (bits | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), rounded)
    return rounded.astype(np.uint32).view(F32)


def bf16_to_bits(x) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns (after RNE rounding)."""

    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_bits_to_f32(bits) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""

    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def fp8_e4m3_round(x) -> np.ndarray:
    """Round float32 to OCP fp8 e4m3fn values (RNE), returned as float32.

    Inputs must already be clamped to [-448, 448], as ``moe_runtime.py:232``
    does before the cast.  Normal range keeps 3 mantissa bits; below 2^-6 the
    quantum is 2^-9 (subnormals).
    """

    a = np.asarray(x, dtype=F32)
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 20) & 1
    normal = ((bits + 0x7FFFF + lsb) & 0xFFF00000).astype(np.uint32).view(F32)
    sub = (np.rint(a.astype(np.float64) * 512.0) / 512.0).astype(F32)
    out = np.where(np.abs(a) < F32(2.0**-6), sub, normal)
    return out.astype(F32)


def fp8_e4m3_encode(v) -> np.ndarray:
    """float32 values already representable in e4m3fn -> uint8 codes."""

    a = np.asarray(v, dtype=np.float64)
    sign = (np.signbit(a)).astype(np.uint8) << 7
    mag = np.abs(a)
    code = np.zeros(a.shape, dtype=np.uint8)
    nz = mag > 0
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(nz, mag, 1.0))).astype(np.int64)
    is_normal = nz & (e >= -6)
    man_n = np.rint((mag / np.exp2(e.astype(np.float64)) - 1.0) * 8.0).astype(np.int64)
    code_n = ((e + 7) << 3) | man_n
    man_s = np.rint(mag * 512.0).astype(np.int64)
    code = np.where(is_normal, code_n, np.where(nz, man_s, 0)).astype(np.uint8)
    return (code | sign).astype(np.uint8)


def fp8_e4m3_decode(codes) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 (0x7F/0xFF decode to NaN)."""

    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(F32)


# ---------------------------------------------------------------------------
# Elementary fp32 functions with a fixed operation sequence.
#
# Every step is one IEEE float32 operation (no fused multiply-add), so the HIP
# router kernel, which spells out the same sequence, reproduces these bits.
# exp: Cody & Waite range reduction (W. J. Cody, W. Waite, "Software Manual for
# the Elementary Functions", 1980) with a degree-7 Taylor polynomial.
# log: mantissa in [sqrt(1/2), sqrt(2)) and the atanh series
# log(m) = 2*atanh((m-1)/(m+1)).  log1p: Goldberg's compensation
# (D. Goldberg, "What every computer scientist should know about floating-point
# arithmetic", 1991, Theorem 4).
# ---------------------------------------------------------------------------

_LOG2E = F32(1.4426950408889634)
_LN2_HI = F32(0.693359375)
_LN2_LO = F32(-2.12194440e-4)
_EXP_C = [F32(1.0 / math.factorial(i)) for i in range(8)]  # 1, 1, 1/2, ..., 1/5040
_SQRT2 = F32(1.41421356237)
_LOG_C = [F32(1.0 / 3.0), F32(1.0 / 5.0), F32(1.0 / 7.0), F32(1.0 / 9.0)]


def exp_f32(x) -> np.ndarray:
    """exp(x) in float32; 0 below 2^-126 (no subnormal results), inf above 2^128."""

    x = np.minimum(np.maximum(np.asarray(x, dtype=F32), F32(-110.0)), F32(100.0))
    n = np.rint(x * _LOG2E).astype(F32)
    r = (x - n * _LN2_HI) - n * _LN2_LO
    p = _EXP_C[7]
    for c in reversed(_EXP_C[:7]):
        p = p * r + c
    ni = n.astype(np.int32)
    scale_bits = (np.clip(ni, -126, 127) + 127).astype(np.uint32) << np.uint32(23)
    out = (p * scale_bits.view(F32)).astype(F32)
    out = np.where(ni > 127, F32(np.inf), out)
    out = np.where(ni <= -126, F32(0.0), out)
    return out.astype(F32)


def log_f32(x) -> np.ndarray:
    """log(x) for finite normal x >= 1 (the only domain the router needs)."""

    x = np.asarray(x, dtype=F32)
    bits = x.view(np.uint32)
    e = ((bits >> np.uint32(23)) & np.uint32(0xFF)).astype(np.int32) - 127
    m = ((bits & np.uint32(0x7FFFFF)) | np.uint32(0x3F800000)).view(F32)
    big = m > _SQRT2
    m = np.where(big, m * F32(0.5), m).astype(F32)
    e = np.where(big, e + 1, e)
    s = (m - F32(1.0)) / (m + F32(1.0))
    s2 = s * s
    t = _LOG_C[3]
    for c in (_LOG_C[2], _LOG_C[1], _LOG_C[0]):
        t = t * s2 + c
    t = t * s2
    log_m = (s + s * t) * F32(2.0)
    ef = e.astype(F32)
    return (ef * _LN2_HI + (ef * _LN2_LO + log_m)).astype(F32)


def log1p_f32(u) -> np.ndarray:
    """log(1+u) for u >= 0."""

    u = np.asarray(u, dtype=F32)
    w = (u + F32(1.0)).astype(F32)
    one = w == F32(1.0)
    safe_w = np.where(one, F32(2.0), w)
    denom = (safe_w - F32(1.0)).astype(F32)
    val = log_f32(safe_w) * (np.where(one, F32(1.0), u) / denom)
    return np.where(one, u, val).astype(F32)


def sigmoid_f32(x) -> np.ndarray:
    """``Tensor.sigmoid`` (``reference/inference/model.py:568-569``) as 1/(1+exp(-x))."""

    x = np.asarray(x, dtype=F32)
    return (F32(1.0) / (F32(1.0) + exp_f32(-x))).astype(F32)


def sqrtsoftplus_f32(x) -> np.ndarray:
    """sqrt(softplus(x)) with torch's threshold 20 (``moe_forward.py:80``)."""

    x = np.asarray(x, dtype=F32)
    sp = np.where(x > F32(20.0), x, log1p_f32(exp_f32(np.minimum(x, F32(20.0)))))
    return np.sqrt(sp.astype(F32)).astype(F32)


def softmax_f32(x) -> np.ndarray:
    """Row softmax (``model.py:566-567``) with a fixed summation tree.

    Expert e is owned by lane e % 64 of a 64-lane wavefront; each lane sums its
    experts in ascending order, then the lanes combine with a xor butterfly of
    distance 32, 16, 8, 4, 2, 1 (every lane ends with the same bits).
    """

    x = np.asarray(x, dtype=F32)
    t, e = x.shape
    m = x.max(axis=1, keepdims=True)
    v = exp_f32(x - m)
    partial = np.zeros((t, 64), dtype=F32)
    for j in range(e):
        partial[:, j % 64] = partial[:, j % 64] + v[:, j]
    lanes = np.arange(64)
    for off in (32, 16, 8, 4, 2, 1):
        partial = (partial + partial[:, lanes ^ off]).astype(F32)
    return (v / partial[:, :1]).astype(F32)


def route_scores(logits, score_func: int) -> np.ndarray:
    """Scores of ``Gate.forward`` (``model.py:565-571``)."""

    if score_func == SCORE_SIGMOID:
        return sigmoid_f32(logits)
    if score_func == SCORE_SOFTMAX:
        return softmax_f32(logits)
    if score_func == SCORE_SQRTSOFTPLUS:
        return sqrtsoftplus_f32(logits)
    raise ValueError(f"unknown score_func {score_func}")


# ---------------------------------------------------------------------------
# Router top-k (a1)
# ---------------------------------------------------------------------------


def _order_key(values: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 image of float32 values (-0.0 sorts below +0.0)."""

    bits = np.ascontiguousarray(values, dtype=F32).view(np.uint32)
    neg = (bits >> np.uint32(31)).astype(bool)
    return np.where(neg, ~bits, bits | np.uint32(0x80000000)).astype(np.uint32)


@dataclass(frozen=True)
class RouteResult:
    ids: np.ndarray  # int32 [T, k]
    weights: np.ndarray  # float32 [T, k]
    margin: np.ndarray  # float32 [T]
    scores: np.ndarray  # float32 [T, E] unbiased
    selection_ids: np.ndarray  # int32 [T, k+1] (or [T, k] when k == E)
    selection_scores: np.ndarray  # float32 [T, k+1]


def route_topk(
    logits,
    topk: int,
    *,
    score_func: int = SCORE_SIGMOID,
    bias=None,
    route_scale: float = 1.0,
) -> RouteResult:
    """``Gate.forward`` (``reference/inference/model.py:564-584``) with the
    boundary outputs of ``gate_forward_with_boundary`` (``moe_forward.py:80-87``).

    Selection orders experts by (biased score descending, expert id ascending).
    Weights gather the *unbiased* scores; for non-softmax scores they are
    divided by their sequential sum (selection order), then multiplied by
    ``route_scale``.  margin = sel[k-1] - sel[k] (0 when k == E).
    """

    logits = np.asarray(logits, dtype=F32)
    t, e = logits.shape
    if not 0 < topk <= e:
        raise ValueError("topk must be in [1, experts]")
    scores = route_scores(logits, score_func)
    sel = scores if bias is None else (scores + np.asarray(bias, dtype=F32)[None, :]).astype(F32)
    depth = min(topk + 1, e)
    key = _order_key(sel)
    comp = ((~key).astype(np.uint64) << np.uint64(32)) | np.arange(e, dtype=np.uint64)[None, :]
    order = np.argsort(comp, axis=1, kind="stable")[:, :depth].astype(np.int32)
    sel_sorted = np.take_along_axis(sel, order, axis=1)
    ids = order[:, :topk].copy()
    if depth > topk:
        margin = (sel_sorted[:, topk - 1] - sel_sorted[:, topk]).astype(F32)
    else:
        margin = np.zeros(t, dtype=F32)
    w = np.take_along_axis(scores, ids, axis=1).astype(F32)
    if score_func != SCORE_SOFTMAX:
        total = w[:, 0].copy()
        for j in range(1, topk):
            total = (total + w[:, j]).astype(F32)
        w = (w / total[:, None]).astype(F32)
    w = (w * F32(route_scale)).astype(F32)
    return RouteResult(ids, w, margin, scores, order, sel_sorted.astype(F32))


def hash_route(logits, tid2eid, input_ids, *, route_scale: float = 1.0) -> RouteResult:
    """``hash_gate_forward`` (``moe_forward.py:186-231``): ids from the token
    table, weights from sqrt-softplus scores, renormalised, times route_scale."""

    logits = np.asarray(logits, dtype=F32)
    scores = sqrtsoftplus_f32(logits)
    ids = np.asarray(tid2eid)[np.asarray(input_ids)].astype(np.int32)
    w = np.take_along_axis(scores, ids, axis=1).astype(F32)
    total = w[:, 0].copy()
    for j in range(1, ids.shape[1]):
        total = (total + w[:, j]).astype(F32)
    w = ((w / total[:, None]).astype(F32) * F32(route_scale)).astype(F32)
    zero = np.zeros(ids.shape[0], dtype=F32)
    return RouteResult(ids, w, zero, scores, ids, w)


# ---------------------------------------------------------------------------
# Block size policy and alignment (a3, a4)
# ---------------------------------------------------------------------------


def marlin_block_size_m(rows: int, topk: int, experts: int, act_itemsize: int = 2) -> int:
    """``_marlin_block_size_m`` (``runtime/dsv4_direct/moe_runtime.py:276-300``)."""

    if rows <= 0 or topk <= 0 or experts <= 0:
        raise ValueError("rows, topk and experts must be positive")
    selected = 64
    for candidate in (8, 16, 32, 48, 64):
        if rows * topk / experts / candidate < 0.9:
            selected = candidate
            break
    if act_itemsize == 1:
        selected = max(selected, 16)
    return selected


def max_padded_tokens(num_assignments: int, num_experts: int, block_size: int) -> int:
    """``max_padded_tokens`` (``deterministic_moe_align.py:17-32``)."""

    for value in (num_assignments, num_experts, block_size):
        if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
            raise ValueError("arguments must be positive integers")
    maximum = num_assignments + num_experts * (block_size - 1)
    if num_assignments < num_experts:
        maximum = min(num_assignments * block_size, maximum)
    return maximum


@dataclass(frozen=True)
class AlignResult:
    sorted_token_ids: np.ndarray  # int32 [cap]
    expert_ids: np.ndarray  # int32 [ceil(cap/bs)]
    num_tokens_post_padded: int


def moe_align(ids, block_size: int, num_experts: int) -> AlignResult:
    """Closed form of ``deterministic_moe_align_block_size``
    (``deterministic_moe_align.py:93-133``): stable expert-major order by flat
    index, each expert run padded to a multiple of ``block_size`` with the
    sentinel ``T*k``, per-block expert ids, -1 past the padded total."""

    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    a = flat.size
    if a == 0:
        raise ValueError("empty route ids")
    if flat.min() < 0 or flat.max() >= num_experts:
        raise ValueError("route id out of range")
    cap = max_padded_tokens(a, num_experts, block_size)
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    dense_offsets = np.cumsum(counts) - counts
    padded = (counts + block_size - 1) // block_size * block_size
    padded_ends = np.cumsum(padded)
    padded_offsets = padded_ends - padded
    order = np.argsort(flat, kind="stable")
    sorted_experts = flat[order]
    ranks = np.arange(a, dtype=np.int64) - dense_offsets[sorted_experts]
    positions = padded_offsets[sorted_experts] + ranks
    sorted_ids = np.full(cap, a, dtype=np.int32)
    sorted_ids[positions] = order.astype(np.int32)
    nblocks = (cap + block_size - 1) // block_size
    starts = np.arange(nblocks, dtype=np.int64) * block_size
    total = int(padded_ends[-1])
    block_experts = np.searchsorted(padded_ends, starts, side="right")
    expert_ids = np.where(starts < total, block_experts, -1).astype(np.int32)
    return AlignResult(sorted_ids, expert_ids, total)


def moe_align_bruteforce(ids, block_size: int, num_experts: int) -> AlignResult:
    """List restatement of ``fixed_b240_alignment_oracle``
    (``fixed_moe_align.py:434-456``), generalised over shape/E/block size."""

    flat = [int(v) for v in np.asarray(ids).reshape(-1).tolist()]
    a = len(flat)
    cap = max_padded_tokens(a, num_experts, block_size)
    sentinel = a
    sorted_values: list[int] = []
    expert_values: list[int] = []
    for expert in range(num_experts):
        matches = [i for i, r in enumerate(flat) if r == expert]
        if not matches:
            continue
        padded = (len(matches) + block_size - 1) // block_size * block_size
        sorted_values.extend(matches)
        sorted_values.extend([sentinel] * (padded - len(matches)))
        expert_values.extend([expert] * (padded // block_size))
    total = len(sorted_values)
    nblocks = (cap + block_size - 1) // block_size
    sorted_values.extend([sentinel] * (cap - len(sorted_values)))
    expert_values.extend([-1] * (nblocks - len(expert_values)))
    return AlignResult(
        np.asarray(sorted_values, dtype=np.int32),
        np.asarray(expert_values, dtype=np.int32),
        total,
    )


# ---------------------------------------------------------------------------
# Weight formats (a5)
# ---------------------------------------------------------------------------

FP4_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)


def pack_int4_rows(q) -> np.ndarray:
    """int values in [-8, 7], shape [N, K] -> uint8 [N, K/2]; the low nibble
    holds the even K index (the checkpoint convention of ``moe_forward.py:126-131``),
    nibbles are two's complement."""

    q = np.asarray(q)
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("int4 values must lie in [-8, 7]")
    nib = (q.astype(np.int16) & 0xF).astype(np.uint8)
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)


_NIBBLE_VALUES = np.array([v if v < 8 else v - 16 for v in range(16)], dtype=np.int8)


def unpack_int4_rows(packed) -> np.ndarray:
    """uint8 [N, K/2] -> int8 [N, K] (inverse of ``pack_int4_rows``)."""

    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = _NIBBLE_VALUES[p & 0xF]
    out[:, 1::2] = _NIBBLE_VALUES[p >> 4]
    return out


EXACT_AMPLIFICATION = 2.0 ** 64


def running_sum_amplification(scale_bits) -> np.ndarray:
    """Per row of int4-g128 group scales (bf16 bits [.., n, k/128]): the
    largest factor max_g (s_0 + ... + s_g) / s_g by which the W4A16 prefill
    kernels' running sum (each accumulator kept divided by the current
    group's scale) can exceed the largest partial sum, in float64.  Rows above
    ``EXACT_AMPLIFICATION`` need exact per-group scaling (the rule of
    ``pack_exact_flag_kernel``)."""

    s = np.abs(bf16_bits_to_f32(np.asarray(scale_bits)).astype(np.float64))
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        return (np.cumsum(s, axis=-1) / s).max(axis=-1)


def needs_exact_scaling(scale_bits) -> np.ndarray:
    """Per matrix (the leading axes of ``scale_bits`` [.., n, k/128]): does any
    row's running-sum amplification exceed 2^64 (or is it not finite)?"""

    amp = running_sum_amplification(scale_bits)
    return ~(amp <= EXACT_AMPLIFICATION).all(axis=-1)


def dequant_int4_g128(packed, scale_bits, group: int = 128) -> np.ndarray:
    """W[n, k] = q[n, k] * s[n, k // group] in float32 (exact).

    ``scale_bits`` are bf16 bit patterns (uint16) of shape [N, K/group].  This is
    the int4-g128 instantiation of the reference's "4-bit code -> value x group
    scale" dequant (``moe_forward.py:126-155``)."""

    q = unpack_int4_rows(packed).astype(F32)
    n, k = q.shape
    s = bf16_bits_to_f32(scale_bits).reshape(n, k // group)
    return (q.reshape(n, k // group, group) * s[:, :, None]).reshape(n, k).astype(F32)


def decode_e8m0(codes) -> np.ndarray:
    """``decode_e8m0_scale_for_oracle`` (``weight_only_linear.py:503-513``):
    byte 0 -> 2^-127, byte b -> 2^(b-127); 255 is reserved (rejected)."""

    c = np.asarray(codes, dtype=np.uint8)
    if (c == 255).any():
        raise ValueError("reserved E8M0 byte 255")
    bits = np.where(c == 0, np.uint32(1 << 22), c.astype(np.uint32) << np.uint32(23))
    return bits.astype(np.uint32).view(F32)


def dequant_mxfp4(packed, scale_codes) -> np.ndarray:
    """``dequant_mxfp4`` (``moe_forward.py:126-155``): E2M1 codes, low nibble =
    even K, one E8M0 scale per 32 K."""

    p = np.asarray(packed, dtype=np.uint8)
    table = np.asarray(FP4_VALUES, dtype=F32)
    vals = np.empty((p.shape[0], p.shape[1] * 2), dtype=F32)
    vals[:, 0::2] = table[p & 0xF]
    vals[:, 1::2] = table[p >> 4]
    s = decode_e8m0(scale_codes)
    return (vals.reshape(p.shape[0], -1, 32) * s[:, :, None]).reshape(vals.shape).astype(F32)


# ---------------------------------------------------------------------------
# Expert FFN, combine and shared expert (a7-a11)
# ---------------------------------------------------------------------------


def _silu(g: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g gives silu = -0
        return (g / (F32(1.0) + np.exp(-g.astype(F32)))).astype(F32)


def _swiglu(g: np.ndarray, u: np.ndarray, clamp_limit: float) -> np.ndarray:
    """``Expert.forward`` activation (``model.py:598-603``)."""

    if clamp_limit > 0:
        u = np.clip(u, -F32(clamp_limit), F32(clamp_limit))
        g = np.minimum(g, F32(clamp_limit))
    return (_silu(g) * u).astype(F32)


def swiglu_f32(g, u, clamp_limit: float) -> np.ndarray:
    """The expert activation in fp32 (``model.py:598-603``), as ``moe_fp32``
    applies it: clamp (when ``clamp_limit`` > 0), then SiLU(gate) * up."""

    return _swiglu(np.asarray(g, dtype=F32), np.asarray(u, dtype=F32), clamp_limit)


class ExpertSource:
    """Accessor for int4-g128 experts in the canonical layout.

    ``w13_packed`` [E', 2I, H/2] u8, ``w13_scale`` [E', 2I, H/128] u16 (bf16 bits),
    ``w2_packed`` [E', H, I/2] u8, ``w2_scale`` [E', H, I/128] u16.  Rows
    [0, I) of w13 are the gate (w1), rows [I, 2I) the up projection (w3)
    (``experiments/A3F-marlin-moe-flash/common.py:7-8``).  Index E (if present)
    is the shared expert.
    """

    def __init__(self, w13_packed, w13_scale, w2_packed, w2_scale, group: int = 128):
        self.w13_packed = w13_packed
        self.w13_scale = w13_scale
        self.w2_packed = w2_packed
        self.w2_scale = w2_scale
        self.group = group

    def w13(self, e: int) -> np.ndarray:
        return dequant_int4_g128(np.asarray(self.w13_packed[e]), np.asarray(self.w13_scale[e]), self.group)

    def w2(self, e: int) -> np.ndarray:
        return dequant_int4_g128(np.asarray(self.w2_packed[e]), np.asarray(self.w2_scale[e]), self.group)


class MXFP4ExpertSource(ExpertSource):
    """Accessor for MXFP4 experts in the checkpoint layout (the reference's
    routed-expert format, ``moe_forward.py:126-155``): ``w13_packed``
    [E', 2I, H/2] u8 E2M1 codes (low nibble = even k), ``w13_scale``
    [E', 2I, H/32] u8 E8M0, ``w2_packed`` [E', H, I/2], ``w2_scale`` [E', H, I/32].
    Dequantisation is ``dequant_mxfp4`` (pinned by the FP4 table and E8M0 KATs)."""

    def __init__(self, w13_packed, w13_scale, w2_packed, w2_scale):
        super().__init__(w13_packed, w13_scale, w2_packed, w2_scale, group=32)

    def w13(self, e: int) -> np.ndarray:
        return dequant_mxfp4(np.asarray(self.w13_packed[e]), np.asarray(self.w13_scale[e]))

    def w2(self, e: int) -> np.ndarray:
        return dequant_mxfp4(np.asarray(self.w2_packed[e]), np.asarray(self.w2_scale[e]))


def moe_fp32(
    x,
    ids,
    weights,
    experts: ExpertSource,
    *,
    shared_index: int | None = None,
    clamp_limit: float = 0.0,
    rows=None,
    workers: int = 1,
) -> np.ndarray:
    """fp32 dequant oracle of the MoE layer (``a3_numerics.py:56-91``;
    official ``MoE.forward``, ``model.py:629-644``): per expert, gate/up in fp32,
    clamp, SiLU*up, times the route weight (on the w2 input, ``model.py:604-606``),
    w2, accumulate in fp32; plus the shared expert with weight 1.

    ``rows`` optionally restricts the output to a subset of token rows (each
    token's output depends only on its own row), returning [len(rows), H].
    ``workers`` > 1 dequantises and multiplies the experts on a thread pool
    (numpy releases the GIL); the per-expert results are added in expert order
    either way.
    """

    x = np.asarray(x, dtype=F32)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=F32)
    if rows is not None:
        rows = np.asarray(rows)
        x, ids, weights = x[rows], ids[rows], weights[rows]
    t, h = x.shape
    y = np.zeros((t, h), dtype=F32)

    def one_expert(e):
        tok, kk = np.nonzero(ids == e)
        w13 = experts.w13(int(e))
        inter = w13.shape[0] // 2
        xe = x[tok]
        g = xe @ w13[:inter].T
        u = xe @ w13[inter:].T
        act = _swiglu(g, u, clamp_limit) * weights[tok, kk][:, None]
        return tok, act.astype(F32) @ experts.w2(int(e)).T

    present = np.unique(ids)
    if workers > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=workers) as pool:
            parts = pool.map(one_expert, present)
            for tok, part in parts:
                y[tok] += part
    else:
        for e in present:
            tok, part = one_expert(e)
            y[tok] += part
    if shared_index is not None:
        w13 = experts.w13(shared_index)
        inter = w13.shape[0] // 2
        act = _swiglu(x @ w13[:inter].T, x @ w13[inter:].T, clamp_limit)
        y += act @ experts.w2(shared_index).T
    return y.astype(F32)


# The bf16 casts of the reference's torch path, by name.  Each entry is
# ``bf16_round``; the table exists so a CPU test can drop one rounding (plant
# an op-order mistake in this oracle) and show that the comparison against
# torch's own bf16 operations detects it.
BF16_CASTS = {
    name: bf16_round
    for name in ("input", "weight", "gemm1_out", "hidden", "gemm2_out", "routed_sum", "shared_gemm1_out",
                 "shared_hidden", "shared_out", "output")
}


def _cast(name: str, x) -> np.ndarray:
    return BF16_CASTS[name](x)


def moe_bf16_mirror(
    x,
    ids,
    weights,
    experts: ExpertSource,
    *,
    shared_index: int | None = None,
    clamp_limit: float = 0.0,
    rows=None,
    workers: int = 1,
) -> np.ndarray:
    """Op-order mirror of the reference's torch MoE path (bf16 output).

    ``DenseRoutedExecutor.__call__`` (``ops/dense_moe.py:289-354``): dequantize
    to bf16 (value * scale rounded to bf16, the int4 analogue of
    ``dequant_mxfp4_bf16`` ``:53-68``), bf16 GEMM with fp32 accumulation and a
    bf16 result, fp32 clamp/SiLU*up, bf16 cast, bf16 w2 GEMM, times the route
    weight in fp32, sum over k in row order, bf16.  Then the shared expert
    (``moe_runtime.py:246-263``) and the bf16 add with fp32 opmath
    (``moe_runtime.py:1873``).  Returns float32 values on the bf16 grid.
    ``workers`` > 1 runs the experts on a thread pool (numpy releases the GIL).
    """

    x = _cast("input", np.asarray(x, dtype=F32))
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=F32)
    if rows is not None:
        rows = np.asarray(rows)
        x, ids, weights = x[rows], ids[rows], weights[rows]
    t, h = x.shape
    k = ids.shape[1]
    contrib = np.zeros((t, k, h), dtype=F32)

    def one_expert(e):
        tok, kk = np.nonzero(ids == e)
        w13 = _cast("weight", experts.w13(int(e)))
        inter = w13.shape[0] // 2
        proj = _cast("gemm1_out", x[tok] @ w13.T)
        hid = _cast("hidden", _swiglu(proj[:, :inter], proj[:, inter:], clamp_limit))
        out = _cast("gemm2_out", hid @ _cast("weight", experts.w2(int(e))).T)
        contrib[tok, kk] = out * weights[tok, kk][:, None]

    if workers > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=workers) as pool:
            list(pool.map(one_expert, np.unique(ids)))
    else:
        for e in np.unique(ids):
            one_expert(e)
    routed = contrib[:, 0].copy()
    for j in range(1, k):
        routed = (routed + contrib[:, j]).astype(F32)
    routed = _cast("routed_sum", routed)
    if shared_index is None:
        return routed
    w13 = _cast("weight", experts.w13(shared_index))
    inter = w13.shape[0] // 2
    proj_g = _cast("shared_gemm1_out", x @ w13[:inter].T)
    proj_u = _cast("shared_gemm1_out", x @ w13[inter:].T)
    hid = _cast("shared_hidden", _swiglu(proj_g, proj_u, clamp_limit))
    shared = _cast("shared_out", hid @ _cast("weight", experts.w2(shared_index)).T)
    return _cast("output", routed + shared)


# ---------------------------------------------------------------------------
# W4A8 (a12) and W8A16 (a13)
# ---------------------------------------------------------------------------


def act_quant_per_token_fp8(x) -> tuple[np.ndarray, np.ndarray]:
    """Per-token fp8 quant (``moe_runtime.py:229-232``):
    s = max(amax, 1e-12) / 448; q = e4m3(clamp(x / s, -448, 448)).
    Returns (q as float32 values on the e4m3 grid, s float32 [T, 1])."""

    xf = np.asarray(x, dtype=F32)
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    s = (np.maximum(amax, F32(1e-12)) / F32(448.0)).astype(F32)
    q = fp8_e4m3_round(np.clip(xf / s, F32(-448.0), F32(448.0)))
    return q.astype(F32), s


def moe_w4a8_f32(
    x,
    ids,
    weights,
    experts: ExpertSource,
    *,
    shared_index: int | None = None,
    clamp_limit: float = 0.0,
    rows=None,
) -> np.ndarray:
    """W4A8 layer oracle: activations into each expert GEMM are quantized per
    row to fp8 e4m3 (``moe_runtime.py:207-235``; Marlin ``input_dtype=fp8``
    quantizes the w13 input and the intermediate), weights int4-g128, fp32
    accumulation, fp32 SwiGLU and combine."""

    x = np.asarray(x, dtype=F32)
    ids = np.asarray(ids)
    weights = np.asarray(weights, dtype=F32)
    if rows is not None:
        rows = np.asarray(rows)
        x, ids, weights = x[rows], ids[rows], weights[rows]
    xq, xs = act_quant_per_token_fp8(x)
    xd = (xq * xs).astype(F32)
    t, h = x.shape
    y = np.zeros((t, h), dtype=F32)

    def ffn(xe, e, w):
        w13 = experts.w13(e)
        inter = w13.shape[0] // 2
        act = bf16_round(_swiglu(xe @ w13[:inter].T, xe @ w13[inter:].T, clamp_limit))
        aq, as_ = act_quant_per_token_fp8(act)
        out = (aq * as_) @ experts.w2(e).T
        return out * w

    for e in np.unique(ids):
        tok, kk = np.nonzero(ids == e)
        y[tok] += ffn(xd[tok], int(e), weights[tok, kk][:, None])
    if shared_index is not None:
        y += ffn(xd, shared_index, F32(1.0))
    return y.astype(F32)


def moe_w4a8_mxfp4_f32(
    x,
    ids,
    weights,
    experts: MXFP4ExpertSource,
    *,
    shared_index: int | None = None,
    clamp_limit: float = 0.0,
    rows=None,
) -> np.ndarray:
    """W4A8 over the checkpoint's MXFP4 experts (the reference's W4A8 mode on
    its routed-expert format: ``_fused_marlin_moe(input_dtype=fp8)`` over
    MXFP4 weights with the ``is_a_8bit`` repack, ``ops/marlin_moe.py:197-222``,
    ``moe_runtime.py:207-235``): the ``moe_w4a8_f32`` pipeline -- per-token
    e4m3 x and h, bf16 SwiGLU output, weight on the w2 output -- over the
    exactly dequantised E2M1 * 2^(e-127) weights."""

    if not isinstance(experts, MXFP4ExpertSource):
        raise TypeError("moe_w4a8_mxfp4_f32 takes an MXFP4ExpertSource")
    return moe_w4a8_f32(x, ids, weights, experts, shared_index=shared_index, clamp_limit=clamp_limit, rows=rows)


def automatic_split_k(m: int, n: int, k: int, block_m: int = 32, block_n: int = 64,
                      block_k: int = 128) -> int:
    """``_automatic_split_k`` (``weight_only_linear.py:168-179``)."""

    tiles = -(-m // block_m) * -(-n // block_n)
    k_blocks = k // block_k
    if tiles < 32 and k_blocks >= 32:
        return 4
    if tiles < 96 and k_blocks >= 16:
        return 2
    return 1


def dequant_fp8_block(codes, scale_codes, block: int = 128) -> np.ndarray:
    """``dequant_fp8_block`` (``moe_forward.py:158-176``): FP8 E4M3 codes
    [N, K] times the E8M0 scale of their ``block`` x ``block`` block
    (scale_codes [ceil(N/block), ceil(K/block)]), in float32."""

    c = np.asarray(codes, dtype=np.uint8)
    n, k = c.shape
    s = decode_e8m0(scale_codes)
    if s.shape != (-(-n // block), -(-k // block)):
        raise ValueError(f"FP8 block scale shape {s.shape} does not match weight {c.shape}")
    expanded = np.repeat(np.repeat(s, block, axis=0), block, axis=1)[:n, :k]
    with np.errstate(over="ignore"):  # large scales overflow to inf, as in the reference's fp32 product
        return (fp8_e4m3_decode(c) * expanded).astype(F32)


def w8a16_fp8_linear_f32(a, codes, scale_codes) -> np.ndarray:
    """C = A . bf16(dequant_fp8_block(Q, s))^T in fp32: the FP8 checkpoint path
    of ``weight_only_linear.py:560-598``, which rounds the scaled weight to
    bf16 before the bf16 MMA (fp32 accumulation)."""

    w = bf16_round(dequant_fp8_block(codes, scale_codes))
    return (np.asarray(a, dtype=F32) @ w.T).astype(F32)


def act_quant_block_fp8(x) -> tuple[np.ndarray, np.ndarray]:
    """``_activation_quant_kernel`` (``fp8_linear.py:354-392``): per row and
    128-K block, s = max(amax, 1e-4) * fp32(1/448) in fp32; the E8M0 exponent
    is its biased exponent plus 1 when the mantissa is nonzero (the next power
    of two at or above s), clamped to [1, 254]; q = e4m3(clamp(x / 2^(e-127),
    -448, 448)).  x: float32 values (bf16 / fp16 inputs widen exactly).
    Returns (E4M3 codes uint8 [M, K], E8M0 bytes uint8 [M, K/128])."""

    xf = np.asarray(x, dtype=F32)
    m, k = xf.shape
    if k % 128:
        raise ValueError("k must be a multiple of 128")
    blocks = xf.reshape(m, k // 128, 128)
    amax = np.abs(blocks).max(axis=-1)
    unrounded = (np.maximum(amax, F32(1.0e-4)) * F32(1.0 / 448.0)).astype(F32)
    bits = unrounded.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int64) + ((bits & 0x7FFFFF) != 0)
    e = np.clip(e, 1, 254)
    scale = (e.astype(np.uint32) << np.uint32(23)).view(F32)
    q = np.clip(blocks / scale[..., None], F32(-448.0), F32(448.0)).astype(F32)
    codes = fp8_e4m3_encode(fp8_e4m3_round(q)).reshape(m, k)
    return codes, e.astype(np.uint8)


def block_fp8_gemm_f32(a_codes, a_scale, w_codes, w_scale) -> np.ndarray:
    """``_block_fp8_gemm_kernel`` (``fp8_linear.py:395-424``) in exact-product
    fp32 form: C = sum over 128-K blocks of (A_blk . W_blk^T) * 2^(ea-127) *
    2^(ew-127), accumulated in float64 and returned as float32 (the kernel
    rounds the fp32 sum to bf16).  a_codes E4M3 [M, K], a_scale E8M0
    [M, K/128], w_codes E4M3 [N, K], w_scale E8M0 [ceil(N/128), K/128]."""

    a = fp8_e4m3_decode(a_codes).astype(np.float64)
    w = fp8_e4m3_decode(w_codes).astype(np.float64)
    m, k = a.shape
    n = w.shape[0]
    sa = decode_e8m0(a_scale).astype(np.float64)               # [M, KB]
    sw = decode_e8m0(w_scale).astype(np.float64)               # [NB, KB]
    sw_rows = np.repeat(sw, 128, axis=0)[:n]                   # [N, KB]
    out = np.zeros((m, n), dtype=np.float64)
    for kb in range(k // 128):
        blk = a[:, kb * 128:(kb + 1) * 128] @ w[:, kb * 128:(kb + 1) * 128].T
        out += blk * sa[:, kb:kb + 1] * sw_rows[None, :, kb]
    return out.astype(F32)


def shared_fp8_bf16(x, w1, s1, w3, s3, w2, s2, clamp_limit: float) -> np.ndarray:
    """``prepare_shared_bf16`` + ``shared_bf16_partial``
    (``moe_runtime.py:238-263``) on FP8-block checkpoint weights: the weights
    dequantised and rounded to bf16, then three bf16 linears with fp32
    accumulation -- gate = bf16(x W1^T) clamped above at L, up = bf16(x W3^T)
    clamped to [-L, L], h = bf16(silu(gate) * up), out = bf16(h W2^T) -- as
    float32 values on the bf16 grid.  ``clamp_limit`` 0 disables the clamps
    (this build's convention for the routed experts too)."""

    x = np.asarray(x, dtype=F32)
    wb1 = bf16_round(dequant_fp8_block(w1, s1))
    wb3 = bf16_round(dequant_fp8_block(w3, s3))
    wb2 = bf16_round(dequant_fp8_block(w2, s2))
    gate = bf16_round(x @ wb1.T)
    up = bf16_round(x @ wb3.T)
    h = bf16_round(_swiglu(gate, up, clamp_limit))
    return bf16_round(h @ wb2.T)


def w8a16_linear_f32(a, q_int8, scale_bits) -> np.ndarray:
    """C = A . (Q * s[n])^T in fp32 (the W8A16 closed form of
    ``weight_only_linear.py:560-598`` with int8 per-output-channel weights)."""

    a = np.asarray(a, dtype=F32)
    s = bf16_bits_to_f32(scale_bits).reshape(-1)
    return ((a @ np.asarray(q_int8, dtype=F32).T) * s[None, :]).astype(F32)


# ---------------------------------------------------------------------------
# Parity metrics (a14)
# ---------------------------------------------------------------------------


def error_metrics(observed, reference) -> dict:
    """``error_metrics`` (``moe_forward.py:234-268``): max_abs and rms_rel."""

    o = np.asarray(observed, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    if o.shape != r.shape:
        raise ValueError("shape mismatch")
    if o.size == 0:
        raise ValueError("cannot compare empty tensors")
    if not (np.isfinite(o).all() and np.isfinite(r).all()):
        return {"finite": False, "max_abs": None, "rms_rel": None, "reference_rms": None}
    d = o - r
    ref_rms = float(np.sqrt(np.mean(r * r)))
    return {
        "finite": True,
        "max_abs": float(np.abs(d).max()),
        "rms_rel": float(np.sqrt(np.mean(d * d)) / max(ref_rms, float(np.finfo(np.float32).eps))),
        "reference_rms": ref_rms,
    }


def rel_fro(observed, reference) -> float:
    """``rel_fro`` (``runtime/c2f_dense_moe_gate.py:66-69``): ||o - r|| / ||r||."""

    o = np.asarray(observed, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    return float(np.linalg.norm(o - r) / np.linalg.norm(r))
