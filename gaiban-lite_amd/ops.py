"""Torch-tensor wrappers of the C ABI (device memory and streams only).

Each wrapper checks dtype / device / shape / contiguity of caller-owned
tensors, then launches on the current HIP stream of the tensors' device.  All
arithmetic happens in the HIP kernels of ``libdsv4moe.so``.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import SCORE_FUNCS, call, ptr

GROUP = 128


def _check(name, t, *, dtype, shape=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} shape must be {tuple(shape)}, got {tuple(t.shape)}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device (cuda) tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


PROFILE_INTERVALS = ("route", "align", "row_sums", "stage1_w13", "stage2_w2", "combine")


def profile_begin(max_calls: int, intervals=None) -> None:
    """Start per-kernel HIP-event timing of the next ``max_calls`` layer calls.

    ``intervals`` (names from PROFILE_INTERVALS) limits the events recorded to
    the stamps bounding those intervals (two events per call for one kernel);
    None records all seven stamps."""

    if intervals is None:
        call("dsv4moe_profile_begin", int(max_calls))
        return
    mask = 0
    for name in intervals:
        i = PROFILE_INTERVALS.index(name)  # interval i lies between stamps i and i + 1
        mask |= (1 << i) | (1 << (i + 1))
    call("dsv4moe_profile_begin_stamps", int(max_calls), mask)


def profile_end() -> tuple[dict[str, float], int]:
    """Stop timing; returns (mean ms per timed kernel interval, calls recorded)."""

    import ctypes

    out = (ctypes.c_float * len(PROFILE_INTERVALS))()
    calls = ctypes.c_int32(0)
    call("dsv4moe_profile_end", out, len(PROFILE_INTERVALS), ctypes.byref(calls))
    return {k: float(out[i]) for i, k in enumerate(PROFILE_INTERVALS) if out[i] >= 0.0}, int(calls.value)


def score_func_id(score_func: str | int) -> int:
    if isinstance(score_func, int):
        if score_func not in SCORE_FUNCS.values():
            raise ValueError(f"unknown score_func {score_func}")
        return score_func
    try:
        return SCORE_FUNCS[score_func]
    except KeyError as exc:
        raise ValueError(f"unknown score_func {score_func!r}") from exc


def block_size_m(rows: int, topk: int, experts: int, act_itemsize: int = 2) -> int:
    bs = _lib.load().dsv4moe_block_size_m(rows, topk, experts, act_itemsize)
    if bs < 0:
        raise ValueError("rows, topk and experts must be positive")
    return int(bs)


def route_topk_into(
    logits: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    topk: int,
    score_func: str | int,
    route_scale: float,
    ids: torch.Tensor,
    weights: torch.Tensor,
    margin: torch.Tensor | None = None,
    selection_ids: torch.Tensor | None = None,
    selection_scores: torch.Tensor | None = None,
) -> None:
    if logits.ndim != 2:
        raise ValueError("logits must be [tokens, experts]")
    tokens, experts = logits.shape
    dev = logits.device
    _check("logits", logits, dtype=torch.float32, device=dev)
    if bias is not None:
        _check("bias", bias, dtype=torch.float32, shape=(experts,), device=dev)
    _check("ids", ids, dtype=torch.int32, shape=(tokens, topk), device=dev)
    _check("weights", weights, dtype=torch.float32, shape=(tokens, topk), device=dev)
    if margin is not None:
        _check("margin", margin, dtype=torch.float32, shape=(tokens,), device=dev)
    depth = min(topk + 1, experts)
    if selection_ids is not None:
        _check("selection_ids", selection_ids, dtype=torch.int32, shape=(tokens, depth), device=dev)
    if selection_scores is not None:
        _check("selection_scores", selection_scores, dtype=torch.float32, shape=(tokens, depth), device=dev)
    call(
        "dsv4moe_route_topk", ptr(logits), ptr(bias), tokens, experts, topk,
        score_func_id(score_func), float(route_scale), ptr(ids), ptr(weights), ptr(margin),
        ptr(selection_ids), ptr(selection_scores), _lib.current_stream(dev),
    )


def route_hash_into(
    logits: torch.Tensor,
    tid2eid: torch.Tensor,
    input_ids: torch.Tensor,
    *,
    route_scale: float,
    ids: torch.Tensor,
    weights: torch.Tensor,
    selected_scores: torch.Tensor | None = None,
) -> None:
    tokens, experts = logits.shape
    dev = logits.device
    _check("logits", logits, dtype=torch.float32, device=dev)
    _check("tid2eid", tid2eid, dtype=torch.int64, device=dev)
    _check("input_ids", input_ids, dtype=torch.int64, shape=(tokens,), device=dev)
    topk = tid2eid.shape[1]
    _check("ids", ids, dtype=torch.int32, shape=(tokens, topk), device=dev)
    _check("weights", weights, dtype=torch.float32, shape=(tokens, topk), device=dev)
    if selected_scores is not None:
        _check("selected_scores", selected_scores, dtype=torch.float32, shape=(tokens, topk), device=dev)
    call(
        "dsv4moe_route_hash", ptr(logits), ptr(tid2eid), tid2eid.shape[0], ptr(input_ids),
        tokens, experts, topk, float(route_scale), ptr(ids), ptr(weights), ptr(selected_scores),
        _lib.current_stream(dev),
    )


def gate_logits_into(x: torch.Tensor, weight: torch.Tensor, logits: torch.Tensor) -> None:
    tokens, hidden = x.shape
    experts = weight.shape[0]
    dev = x.device
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("weight", weight, dtype=torch.bfloat16, shape=(experts, hidden), device=dev)
    _check("logits", logits, dtype=torch.float32, shape=(tokens, experts), device=dev)
    call("dsv4moe_gate_logits", ptr(x), ptr(weight), tokens, hidden, experts, ptr(logits),
         _lib.current_stream(dev))


def align_workspace_bytes(tokens: int, topk: int, experts: int) -> int:
    """Scratch bytes of the workgroup-split alignment (0: one workgroup aligns)."""

    return int(_lib.load().dsv4moe_align_workspace_bytes(tokens, topk, experts))


def align_into(
    ids: torch.Tensor,
    *,
    block_size: int,
    num_experts: int,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    workspace: torch.Tensor | None = None,
) -> None:
    """Deterministic alignment; with a ``workspace`` of at least
    ``align_workspace_bytes`` bytes, many ids are aligned by the
    workgroup-split kernels (same output bits)."""

    tokens, topk = ids.shape
    dev = ids.device
    _check("topk_ids", ids, dtype=torch.int32, device=dev)
    _check("sorted_token_ids", sorted_token_ids, dtype=torch.int32, device=dev)
    _check("expert_ids", expert_ids, dtype=torch.int32, device=dev)
    _check("num_tokens_post_padded", num_tokens_post_padded, dtype=torch.int32, shape=(1,), device=dev)
    if workspace is None:
        call(
            "dsv4moe_align", ptr(ids), tokens, topk, num_experts, block_size, ptr(sorted_token_ids),
            sorted_token_ids.numel(), ptr(expert_ids), expert_ids.numel(),
            ptr(num_tokens_post_padded), _lib.current_stream(dev),
        )
        return
    _check("workspace", workspace, dtype=torch.uint8, device=dev)
    call(
        "dsv4moe_align_ws", ptr(ids), tokens, topk, num_experts, block_size, ptr(sorted_token_ids),
        sorted_token_ids.numel(), ptr(expert_ids), expert_ids.numel(),
        ptr(num_tokens_post_padded), ptr(workspace), workspace.numel(), _lib.current_stream(dev),
    )


def pack_int4_g128(canon: torch.Tensor, scales: torch.Tensor, *, gated: bool = False
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """Checkpoint-layout int4 [.., n, k/2] u8 + bf16 scales [.., n, k/128] ->
    pair-interleaved tiles (packed u8 [.., n*k/2], scales bf16 [.., n*k/128]).
    ``gated`` pairs row strip p with strip p of the second half (w13 gate/up)."""

    if canon.ndim == 2:
        canon = canon.unsqueeze(0)
        scales = scales.unsqueeze(0)
        squeeze = True
    else:
        squeeze = False
    batch, n, half_k = canon.shape
    k = half_k * 2
    dev = canon.device
    _check("canon", canon, dtype=torch.uint8, device=dev)
    _check("scales", scales, dtype=torch.bfloat16, shape=(batch, n, k // GROUP), device=dev)
    packed = torch.empty((batch, n * half_k), dtype=torch.uint8, device=dev)
    packed_scales = torch.empty((batch, n * (k // GROUP)), dtype=torch.bfloat16, device=dev)
    call("dsv4moe_pack_int4_g128", ptr(canon), ptr(scales), batch, n, k,
         _lib.PAIR_GATED if gated else _lib.PAIR_PLAIN, ptr(packed), ptr(packed_scales),
         _lib.current_stream(dev))
    if squeeze:
        return packed[0], packed_scales[0]
    return packed, packed_scales


def pack_int4_ratios(packed_scales: torch.Tensor, *, n: int, k: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ratios of consecutive group scales of ``pack_int4_g128`` scales
    (``dsv4moe_pack_int4_ratios``): same shape and element order, element =
    the row's scale of group g-1 over its scale of group g (0 for g = 0).
    The W4A16 prefill kernels read them.  With ``out`` (fp32, the scales'
    shape) the ratios are written there and nothing is allocated."""

    dev = packed_scales.device
    _check("packed_scales", packed_scales, dtype=torch.bfloat16, device=dev)
    if packed_scales.shape[-1] != n * (k // GROUP):
        raise ValueError(f"packed_scales: last dimension {packed_scales.shape[-1]} != n*k/128 = {n * (k // GROUP)}")
    batch = packed_scales.numel() // packed_scales.shape[-1] if packed_scales.ndim > 1 else 1
    if out is None:
        ratios = torch.empty(packed_scales.shape, dtype=torch.float32, device=dev)
    else:
        _check("out", out, dtype=torch.float32, device=dev, shape=tuple(packed_scales.shape))
        ratios = out
    call("dsv4moe_pack_int4_ratios", ptr(packed_scales), batch, n, k, ptr(ratios), _lib.current_stream(dev))
    return ratios


def pack_mxfp4_g32(canon: torch.Tensor, scales: torch.Tensor, *, gated: bool = False, w4a8: bool = False
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """Checkpoint-layout MXFP4 [.., n, k/2] u8 (E2M1, low nibble = even k) +
    E8M0 scales [.., n, k/32] u8 -> tiles (packed u8 [.., n*k/2], scales u8
    [.., n*k/32]) in the tile geometry and pairing of ``pack_int4_g128``.
    ``w4a8`` selects the lane layout of the W4A8 kernels
    (``dsv4moe_pack_mxfp4_g32_w4a8``: one 32-K scale group per lane)."""

    if canon.ndim == 2:
        canon = canon.unsqueeze(0)
        scales = scales.unsqueeze(0)
        squeeze = True
    else:
        squeeze = False
    batch, n, half_k = canon.shape
    k = half_k * 2
    dev = canon.device
    _check("canon", canon, dtype=torch.uint8, device=dev)
    _check("scales", scales, dtype=torch.uint8, shape=(batch, n, k // 32), device=dev)
    packed = torch.empty((batch, n * half_k), dtype=torch.uint8, device=dev)
    packed_scales = torch.empty((batch, n * (k // 32)), dtype=torch.uint8, device=dev)
    call("dsv4moe_pack_mxfp4_g32_w4a8" if w4a8 else "dsv4moe_pack_mxfp4_g32", ptr(canon), ptr(scales), batch, n, k,
         _lib.PAIR_GATED if gated else _lib.PAIR_PLAIN, ptr(packed), ptr(packed_scales),
         _lib.current_stream(dev))
    if squeeze:
        return packed[0], packed_scales[0]
    return packed, packed_scales


def experts_workspace_bytes(tokens: int, topk: int, hidden: int, inter: int, has_shared: bool) -> int:
    return int(_lib.load().dsv4moe_experts_workspace_bytes(tokens, topk, hidden, inter, int(bool(has_shared))))


def experts_w4a8_workspace_bytes(tokens: int, topk: int, hidden: int, inter: int, has_shared: bool) -> int:
    return int(_lib.load().dsv4moe_experts_w4a8_workspace_bytes(tokens, topk, hidden, inter,
                                                                  int(bool(has_shared))))


def w4a8_workspace_views(workspace: torch.Tensor, tokens: int, topk: int, hidden: int, inter: int,
                         has_shared: bool) -> dict[str, torch.Tensor]:
    """Views of the pieces of a W4A8 entry's workspace after a call (the
    layout of ``dsv4moe_experts_w4a8_workspace_bytes``: 256-byte aligned e4m3
    x [T, H], its fp32 row scales [T] and per-128 sums [T, H/128], bf16 h
    [R, I], e4m3 h [R, I], its scales [R] and sums [R, I/128], fp32
    contributions [R, H]; R = T*k (+ T with the shared expert, whose rows
    follow the routed ones)).  For inspection; nothing is copied."""

    rows = tokens * topk + (tokens if has_shared else 0)
    pieces = [("xq", torch.uint8, (tokens, hidden)), ("xscale", torch.float32, (tokens,)),
              ("xsum", torch.float32, (tokens, hidden // GROUP)), ("h", torch.bfloat16, (rows, inter)),
              ("hq", torch.uint8, (rows, inter)), ("hscale", torch.float32, (rows,)),
              ("hsum", torch.float32, (rows, inter // GROUP)), ("contrib", torch.float32, (rows, hidden))]
    views, off = {}, 0
    for name, dtype, shape in pieces:
        n = dtype.itemsize
        for d in shape:
            n *= d
        views[name] = workspace[off:off + n].view(dtype).view(shape)
        off += -(-n // 256) * 256
    if off > workspace.numel():
        raise ValueError(f"workspace of {workspace.numel()} bytes is below the {off} the layout needs")
    return views


def act_quant_fp8_into(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, group_sums: torch.Tensor) -> None:
    """Per-row e4m3 quantisation (q in the fp8 MFMA byte order, see
    ``dsv4moe_act_quant_fp8``)."""

    rows, k = x.shape
    dev = x.device
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("q", q, dtype=torch.uint8, shape=(rows, k), device=dev)
    _check("scale", scale, dtype=torch.float32, shape=(rows,), device=dev)
    _check("group_sums", group_sums, dtype=torch.float32, shape=(rows, k // GROUP), device=dev)
    call("dsv4moe_act_quant_fp8", ptr(x), rows, k, ptr(q), ptr(scale), ptr(group_sums),
         _lib.current_stream(dev))


def experts_w4a8_into(x: torch.Tensor, **kw) -> None:
    """W4A8 counterpart of ``experts_w4a16_into`` (same keywords)."""

    _experts_into("dsv4moe_experts_w4a8", x, **kw)


def experts_w4a8_mxfp4_into(x: torch.Tensor, **kw) -> None:
    """W4A8 over MXFP4 experts (``dsv4moe_experts_w4a8_mxfp4``): same
    keywords as ``experts_w4a16_into`` with ``pack_mxfp4_g32(w4a8=True)``
    weights and E8M0 scales; workspace of ``experts_w4a8_workspace_bytes``."""

    _experts_into("dsv4moe_experts_w4a8_mxfp4", x, **kw)


def experts_w4a16_into(x: torch.Tensor, **kw) -> None:
    _experts_into("dsv4moe_experts_w4a16", x, **kw)


def experts_mxfp4_into(x: torch.Tensor, **kw) -> None:
    """MXFP4 experts (``dsv4moe_experts_mxfp4``); same keywords as
    ``experts_w4a16_into`` with ``pack_mxfp4_g32`` weights and E8M0 scales."""

    _experts_into("dsv4moe_experts_mxfp4", x, **kw)


def _experts_into(
    entry: str,
    x: torch.Tensor,
    *,
    w13q, w13s, w2q, w2s,
    w13r=None, w2r=None,
    experts: int,
    inter: int,
    has_shared: bool,
    route_weights: torch.Tensor,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    block_size: int,
    clamp_limit: float,
    out: torch.Tensor,
    workspace: torch.Tensor,
) -> None:
    tokens, hidden = x.shape
    topk = route_weights.shape[1]
    dev = x.device
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(tokens, hidden), device=dev)
    _check("route_weights", route_weights, dtype=torch.float32, shape=(tokens, topk), device=dev)
    _check("workspace", workspace, dtype=torch.uint8, device=dev)
    ratios = _scale_ratio_args(entry == "dsv4moe_experts_w4a16", w13r, w2r, w13s, w2s, dev)
    call(
        entry, ptr(x), tokens, hidden, inter, experts, topk, ptr(w13q),
        ptr(w13s), ptr(w2q), ptr(w2s), *ratios, int(bool(has_shared)), ptr(route_weights),
        ptr(sorted_token_ids), sorted_token_ids.numel(), ptr(expert_ids),
        ptr(num_tokens_post_padded), block_size, float(clamp_limit), ptr(out), ptr(workspace),
        workspace.numel(), _lib.current_stream(dev),
    )


def _scale_ratio_args(takes_ratios: bool, w13r, w2r, w13s, w2s, dev) -> list:
    """The (w13r, w2r) pointer arguments of the W4A16 entries (fp32, shaped
    as their scales); the other formats take none."""

    if not takes_ratios:
        if w13r is not None or w2r is not None:
            raise ValueError("only the W4A16 entries take scale ratios")
        return []
    if w13r is None or w2r is None:
        raise TypeError("the W4A16 entries need w13r and w2r (pack_int4_ratios of the scales)")
    _check("w13r", w13r, dtype=torch.float32, shape=tuple(w13s.shape), device=dev)
    _check("w2r", w2r, dtype=torch.float32, shape=tuple(w2s.shape), device=dev)
    return [ptr(w13r), ptr(w2r)]


def layer_w4a16_into(
    x: torch.Tensor,
    logits: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    topk: int,
    score_func: str | int,
    route_scale: float,
    w13q, w13s, w2q, w2s,
    w13r=None, w2r=None,
    experts: int,
    inter: int,
    has_shared: bool,
    clamp_limit: float,
    block_size: int,
    ids: torch.Tensor,
    weights: torch.Tensor,
    margin: torch.Tensor | None,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    out: torch.Tensor,
    workspace: torch.Tensor,
    mxfp4: bool = False,
) -> None:
    """The fused layer entry (``dsv4moe_layer_w4a16``, or with ``mxfp4``
    ``dsv4moe_layer_mxfp4`` over the MXFP4 residents)."""

    tokens, hidden = x.shape
    dev = x.device
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("logits", logits, dtype=torch.float32, shape=(tokens, experts), device=dev)
    _check("ids", ids, dtype=torch.int32, shape=(tokens, topk), device=dev)
    _check("weights", weights, dtype=torch.float32, shape=(tokens, topk), device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(tokens, hidden), device=dev)
    _check("workspace", workspace, dtype=torch.uint8, device=dev)
    if bias is not None:
        _check("bias", bias, dtype=torch.float32, shape=(experts,), device=dev)
    ratios = _scale_ratio_args(not mxfp4, w13r, w2r, w13s, w2s, dev)
    call(
        "dsv4moe_layer_mxfp4" if mxfp4 else "dsv4moe_layer_w4a16", ptr(x), ptr(logits), ptr(bias), tokens,
        hidden, inter, experts,
        topk, score_func_id(score_func), float(route_scale), ptr(w13q), ptr(w13s), ptr(w2q),
        ptr(w2s), *ratios, int(bool(has_shared)), float(clamp_limit), block_size, ptr(ids), ptr(weights),
        ptr(margin), ptr(sorted_token_ids), sorted_token_ids.numel(), ptr(expert_ids),
        ptr(num_tokens_post_padded), ptr(out), ptr(workspace), workspace.numel(),
        _lib.current_stream(dev),
    )


def layer_w4a8_into(
    x: torch.Tensor,
    logits: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    topk: int,
    score_func: str | int,
    route_scale: float,
    w13q, w13s, w2q, w2s,
    experts: int,
    inter: int,
    has_shared: bool,
    clamp_limit: float,
    block_size: int,
    ids: torch.Tensor,
    weights: torch.Tensor,
    margin: torch.Tensor | None,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    out: torch.Tensor,
    workspace: torch.Tensor,
    mxfp4: bool = False,
) -> None:
    """The fused W4A8 layer entry (``dsv4moe_layer_w4a8`` over int4 residents,
    or with ``mxfp4`` ``dsv4moe_layer_w4a8_mxfp4`` over MXFP4 residents packed
    for the W4A8 kernels): x is quantised beside the alignment; the workspace
    is ``experts_w4a8_workspace_bytes``."""

    tokens, hidden = x.shape
    dev = x.device
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("logits", logits, dtype=torch.float32, shape=(tokens, experts), device=dev)
    _check("ids", ids, dtype=torch.int32, shape=(tokens, topk), device=dev)
    _check("weights", weights, dtype=torch.float32, shape=(tokens, topk), device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(tokens, hidden), device=dev)
    _check("workspace", workspace, dtype=torch.uint8, device=dev)
    if bias is not None:
        _check("bias", bias, dtype=torch.float32, shape=(experts,), device=dev)
    call(
        "dsv4moe_layer_w4a8_mxfp4" if mxfp4 else "dsv4moe_layer_w4a8", ptr(x), ptr(logits), ptr(bias), tokens,
        hidden, inter, experts, topk, score_func_id(score_func), float(route_scale), ptr(w13q), ptr(w13s),
        ptr(w2q), ptr(w2s), int(bool(has_shared)), float(clamp_limit), block_size, ptr(ids), ptr(weights),
        ptr(margin), ptr(sorted_token_ids), sorted_token_ids.numel(), ptr(expert_ids),
        ptr(num_tokens_post_padded), ptr(out), ptr(workspace), workspace.numel(),
        _lib.current_stream(dev),
    )


def pack_int8(weight: torch.Tensor) -> torch.Tensor:
    """Row-major int8 [n, k] -> tiled uint8 [n*k] (16 rows x 64 K per KiB tile)."""

    if weight.ndim != 2:
        raise ValueError("weight must be [n, k]")
    n, k = weight.shape
    _check("weight", weight, dtype=torch.int8, device=weight.device)
    packed = torch.empty((n * k,), dtype=torch.uint8, device=weight.device)
    call("dsv4moe_pack_int8", ptr(weight), n, k, ptr(packed), _lib.current_stream(weight.device))
    return packed


def pack_fp8(weight: torch.Tensor) -> torch.Tensor:
    """Row-major FP8 E4M3 codes [n, k] (uint8 or float8_e4m3fn) -> the same
    tiled uint8 [n*k] layout as ``pack_int8`` (a byte permutation)."""

    if weight.ndim != 2:
        raise ValueError("weight must be [n, k]")
    if weight.dtype == torch.float8_e4m3fn:
        weight = weight.view(torch.uint8)
    _check("weight", weight, dtype=torch.uint8, device=weight.device)
    return pack_int8(weight.view(torch.int8))


DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.float8_e4m3fn: 3}


def _aligned(t: torch.Tensor, align: int) -> torch.Tensor:
    """``t`` contiguous and starting at an ``align``-byte boundary (a fresh
    copy when a view starts elsewhere)."""

    t = t.contiguous()
    return t if t.data_ptr() % align == 0 else t.clone()


def decode_e8m0(codes: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes (uint8, any shape) -> fp32 of the same shape: 2^(c - 127),
    byte 0 -> 2^-127, byte 255 -> NaN."""

    _check("codes", codes.contiguous(), dtype=torch.uint8)
    out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    call("dsv4moe_decode_e8m0", ptr(codes.contiguous()), codes.numel(), ptr(out), _lib.current_stream(codes.device))
    return out


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """E2M1 codes uint8 [rows, k/2] (low nibble = even K) times decoded fp32
    scales [rows, k/32] -> fp32 [rows, k]."""

    rows, half_k = packed.shape
    packed = _aligned(packed, 16)
    scale = _aligned(scale, 4)
    _check("packed", packed, dtype=torch.uint8)
    _check("scale", scale, dtype=torch.float32, shape=(rows, 2 * half_k // 32), device=packed.device)
    out = torch.empty((rows, 2 * half_k), dtype=torch.float32, device=packed.device)
    call("dsv4moe_dequant_mxfp4", ptr(packed), ptr(scale), rows, 2 * half_k, ptr(out),
         _lib.current_stream(packed.device))
    return out


def dequant_fp8_block(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """A [rows, cols] weight (E4M3FN, bf16, fp16 or fp32) times decoded fp32
    scales [ceil(rows/128), ceil(cols/128)] per 128 x 128 block -> fp32."""

    rows, cols = weight.shape
    if weight.dtype not in DTYPE_CODES:
        raise TypeError(f"weight must be one of {sorted(map(str, DTYPE_CODES))}, got {weight.dtype}")
    weight = _aligned(weight, weight.element_size())
    _check("weight", weight, dtype=weight.dtype)
    scale = _aligned(scale, 4)
    _check("scale", scale, dtype=torch.float32, shape=(-(-rows // 128), -(-cols // 128)), device=weight.device)
    out = torch.empty((rows, cols), dtype=torch.float32, device=weight.device)
    code = DTYPE_CODES[weight.dtype]
    call("dsv4moe_dequant_fp8_block", ptr(weight), code, ptr(scale), rows, cols, ptr(out),
         _lib.current_stream(weight.device))
    return out


def w8a16_split_k(m: int, n: int, k: int) -> int:
    split = int(_lib.load().dsv4moe_w8a16_split_k(m, n, k))
    if split < 1:
        raise ValueError("m, n and k must be positive")
    return split


def w8a16_workspace_bytes(m: int, n: int, split_k: int) -> int:
    return int(_lib.load().dsv4moe_w8a16_workspace_bytes(m, n, split_k))


def _weight_bytes(name: str, wq: torch.Tensor, n: int, k: int, dev) -> tuple[torch.Tensor, int]:
    """A 1-byte weight as uint8 and its layout code: [n, k] (any 1-byte dtype:
    the checkpoint's bytes, row-major) or flat [n*k] uint8 (the tiles of
    ``pack_int8`` / ``pack_fp8``)."""

    if wq.dim() == 2:
        if wq.element_size() != 1:
            raise TypeError(f"{name} must have 1-byte elements, got {wq.dtype}")
        _check(name, wq, dtype=wq.dtype, shape=(n, k), device=dev)
        return wq.view(torch.uint8), _lib.WEIGHT_ROWMAJOR
    _check(name, wq, dtype=torch.uint8, shape=(n * k,), device=dev)
    return wq, _lib.WEIGHT_TILED


def w8a16_linear_into(a: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, out: torch.Tensor,
                      workspace: torch.Tensor | None, *, n: int, split_k: int) -> None:
    """int8 weights with bf16 per-channel scales ``ws`` [n]
    (``dsv4moe_w8a16_linear``); ``wq`` int8 [n, k] row-major or the flat
    ``pack_int8`` tiles."""

    if a.ndim != 2:
        raise ValueError("activation must be [m, k]")
    m, k = a.shape
    dev = a.device
    _check("activation", a, dtype=torch.bfloat16, device=dev)
    wq, layout = _weight_bytes("weight", wq, n, k, dev)
    _check("weight_scale", ws, dtype=torch.bfloat16, shape=(n,), device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(m, n), device=dev)
    ws_bytes = 0
    if workspace is not None:
        _check("workspace", workspace, dtype=torch.float32, device=dev)
        ws_bytes = workspace.numel() * 4
    call("dsv4moe_w8a16_linear", ptr(a), m, n, k, ptr(wq), layout, ptr(ws), int(split_k), ptr(workspace),
         ws_bytes, ptr(out), _lib.current_stream(dev))


def w8a16_fp8_linear_into(a: torch.Tensor, wq: torch.Tensor, ws8: torch.Tensor, out: torch.Tensor,
                          workspace: torch.Tensor | None, *, n: int, split_k: int) -> None:
    """FP8 E4M3 weights with E8M0 128 x 128 block scales ``ws8`` uint8
    [ceil(n/128), k/128] (``dsv4moe_w8a16_fp8_linear``); ``wq`` the
    checkpoint's E4M3 [n, k] as stored, or the flat ``pack_fp8`` tiles."""

    if a.ndim != 2:
        raise ValueError("activation must be [m, k]")
    m, k = a.shape
    dev = a.device
    _check("activation", a, dtype=torch.bfloat16, device=dev)
    wq, layout = _weight_bytes("weight", wq, n, k, dev)
    _check("weight_scale", ws8, dtype=torch.uint8, shape=((n + 127) // 128, k // 128), device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(m, n), device=dev)
    ws_bytes = 0
    if workspace is not None:
        _check("workspace", workspace, dtype=torch.float32, device=dev)
        ws_bytes = workspace.numel() * 4
    call("dsv4moe_w8a16_fp8_linear", ptr(a), m, n, k, ptr(wq), layout, ptr(ws8), int(split_k), ptr(workspace),
         ws_bytes, ptr(out), _lib.current_stream(dev))


_X_DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def act_quant_block_fp8_into(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor) -> None:
    """Per-row, per-128-K block E4M3 quantisation with E8M0 power-of-two
    scales (``dsv4moe_act_quant_block_fp8``); q uint8 [m, k], scale uint8
    [m, k/128]."""

    if x.ndim != 2:
        raise ValueError("x must be [m, k]")
    if x.dtype not in _X_DTYPE_CODES:
        raise TypeError(f"x must be bfloat16, float16 or float32, got {x.dtype}")
    m, k = x.shape
    dev = x.device
    _check("x", x, dtype=x.dtype, device=dev)
    _check("quantized_out", q, dtype=torch.uint8, shape=(m, k), device=dev)
    _check("scale_out", scale, dtype=torch.uint8, shape=(m, k // 128), device=dev)
    call("dsv4moe_act_quant_block_fp8", ptr(x), _X_DTYPE_CODES[x.dtype], m, k, ptr(q), ptr(scale),
         _lib.current_stream(dev))


def block_fp8_split_k(m: int, n: int, k: int) -> int:
    split = int(_lib.load().dsv4moe_block_fp8_split_k(m, n, k))
    if split < 1:
        raise ValueError("m, n and k must be positive")
    return split


def block_fp8_workspace_bytes(m: int, n: int, split_k: int) -> int:
    return int(_lib.load().dsv4moe_block_fp8_workspace_bytes(m, n, split_k))


def block_fp8_gemm_into(a: torch.Tensor, a_scale: torch.Tensor, wq: torch.Tensor, ws8: torch.Tensor,
                        out: torch.Tensor, workspace: torch.Tensor | None, *, n: int, split_k: int) -> None:
    """Block-FP8 W8A8 GEMM (``dsv4moe_block_fp8_gemm``): a E4M3 uint8 [m, k]
    with E8M0 a_scale [m, k/128]; wq W [n, k] (the checkpoint's E4M3 bytes
    as stored, or the flat ``pack_fp8`` tiles) with E8M0 ws8
    [ceil(n/128), k/128]; out bf16 [m, n]."""

    if a.ndim != 2:
        raise ValueError("activation must be [m, k]")
    m, k = a.shape
    dev = a.device
    _check("activation", a, dtype=torch.uint8, device=dev)
    _check("activation_scale", a_scale, dtype=torch.uint8, shape=(m, k // 128), device=dev)
    wq, layout = _weight_bytes("weight", wq, n, k, dev)
    _check("weight_scale", ws8, dtype=torch.uint8, shape=((n + 127) // 128, k // 128), device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(m, n), device=dev)
    ws_bytes = 0
    if workspace is not None:
        _check("workspace", workspace, dtype=torch.float32, device=dev)
        ws_bytes = workspace.numel() * 4
    call("dsv4moe_block_fp8_gemm", ptr(a), ptr(a_scale), m, n, k, ptr(wq), layout, ptr(ws8), int(split_k),
         ptr(workspace), ws_bytes, ptr(out), _lib.current_stream(dev))


def shared_fp8_workspace_bytes(tokens: int, hidden: int, inter: int) -> int:
    return int(_lib.load().dsv4moe_shared_fp8_workspace_bytes(tokens, hidden, inter))


def shared_fp8_add_into(x: torch.Tensor, shared, *, clamp_limit: float, out: torch.Tensor,
                        workspace: torch.Tensor) -> None:
    """out <- bf16(out + shared(x)) with the FP8-block shared expert
    (``ResidentFP8SharedExpert``; ``dsv4moe_shared_fp8_add``)."""

    tokens, hidden = x.shape
    dev = x.device
    inter = shared.intermediate_size
    _check("x", x, dtype=torch.bfloat16, device=dev)
    _check("out", out, dtype=torch.bfloat16, shape=(tokens, hidden), device=dev)
    _check("workspace", workspace, dtype=torch.uint8, device=dev)
    if shared.hidden_size != hidden:
        raise ValueError("shared expert hidden size does not match x")
    call("dsv4moe_shared_fp8_add", ptr(x), tokens, hidden, inter, ptr(shared.w13_q), ptr(shared.w13_s),
         ptr(shared.w2_q), ptr(shared.w2_s), float(clamp_limit), ptr(out), ptr(workspace), workspace.numel(),
         _lib.current_stream(dev))
