"""Grouped expert kernels (W4A16): bf16 layer output against the fp32 dequant
oracle on the same seeded inputs, to max_rel and rel_fro <= 1e-2.

Each token's output depends only on its own row, so full-size configurations
are checked on a subset of token rows (routing, alignment and every kernel
still run over all tokens).
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import ResidentInt4MoEWeights, ops, route_from_logits, synthetic as S
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size
from helpers import DeviceExpertSource, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
_LAYERS: dict = {}


def layer(shape: S.LayerShape, seed: int = 0):
    key = (shape, seed)
    if key not in _LAYERS:
        if len(_LAYERS) >= 2:
            _LAYERS.clear()
            torch.cuda.empty_cache()
        w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=seed, device=DEV)
        res = ResidentInt4MoEWeights.from_checkpoint_layout(
            w13, s13, w2, s2, experts=shape.experts, has_shared=shape.has_shared)
        _LAYERS[key] = (res, DeviceExpertSource(w13, s13, w2, s2))
    return _LAYERS[key]


def run_experts(shape, x, ids, weights, *, block_size=None, clamp=0.0):
    res, _ = layer(shape)
    t = x.shape[0]
    bs = block_size or ops.block_size_m(t, shape.topk, shape.experts)
    align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=shape.experts)
    out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.experts_workspace_bytes(t, shape.topk, shape.hidden, shape.inter,
                                                 shape.has_shared), dtype=torch.uint8, device=DEV)
    ops.experts_w4a16_into(
        x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
        experts=shape.experts,
        inter=shape.inter, has_shared=shape.has_shared, route_weights=weights,
        sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
        num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=clamp,
        out=out, workspace=ws)
    torch.cuda.synchronize()
    return out


def check_layer(shape, t, *, rows=None, block_size=None, clamp=0.0, x_scale=1.0, seed=1,
                score="sigmoid", ids=None):
    print(f"[experts] E={shape.experts} H={shape.hidden} I={shape.inter} k={shape.topk} T={t} "
          f"bs={block_size} clamp={clamp} x_scale={x_scale}", flush=True)
    x = (S.make_hidden(t, shape.hidden, seed=seed, device=DEV).float() * x_scale).to(torch.bfloat16)
    logits = S.make_logits(t, shape.experts, seed=seed + 1, device=DEV)
    r = route_from_logits(logits, topk=shape.topk, score_func=score)
    route_ids, route_w = r.routing_ids, r.routing_weights
    if ids is not None:
        route_ids = ids
    out = run_experts(shape, x, route_ids, route_w, block_size=block_size, clamp=clamp)
    _, src = layer(shape)
    rows = np.arange(t) if rows is None else np.asarray(rows)
    ref = O.moe_fp32(to_np_f32(x), route_ids.cpu().numpy(), route_w.cpu().numpy(), src,
                     shared_index=shape.experts if shape.has_shared else None,
                     clamp_limit=clamp, rows=rows)
    got = to_np_f32(out)[rows]
    err = assert_moe_close(got, ref, what=f"T={t}")
    print(f"    {err}", flush=True)
    return got, ref


def test_tiny_config_full():
    check_layer(S.TINY, 64)


def test_tiny_config_matches_bf16_mirror_order_of_magnitude():
    got, ref = check_layer(S.TINY, 64, seed=3)
    x = S.make_hidden(64, S.TINY.hidden, seed=3, device=DEV)
    r = route_from_logits(S.make_logits(64, S.TINY.experts, seed=4, device=DEV), topk=2)
    mirror = O.moe_bf16_mirror(to_np_f32(x), r.routing_ids.cpu().numpy(),
                               r.routing_weights.cpu().numpy(), layer(S.TINY)[1])
    # the reference torch path itself sits at the same distance from the fp32 oracle
    assert_moe_close(mirror, ref, what="bf16 mirror vs fp32 oracle")


@pytest.mark.parametrize("bs", [8, 16, 32, 48, 64])
def test_every_block_size_kernel(bs):
    check_layer(S.TINY, 200, block_size=bs, seed=5)


@pytest.mark.parametrize("clamp,x_scale", [(10.0, 1.0), (10.0, 8.0), (2.0, 4.0)])
def test_clamp(clamp, x_scale):
    check_layer(S.TINY, 64, clamp=clamp, x_scale=x_scale, seed=7)


def test_tiny_shared_expert_layout():
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    check_layer(shape, 50, seed=9)


@pytest.mark.parametrize("shared", [False, True])
def test_topk_above_one_combine_batch(shared):
    """Ten slots per token: the combine reads them in two batches of loads."""
    shape = S.LayerShape(experts=16, hidden=1024, inter=512, topk=10, has_shared=shared)
    check_layer(shape, 40, seed=13)


@pytest.mark.parametrize("shared", [False, True])
def test_topk_above_one_combine_batch_sums_in_slot_order(shared):
    """The combine's adds, bit for bit: slot 0, then slots 1..k-1 in order,
    then the shared row, in fp32, one bf16 rounding.  The fp32 contributions
    are read back from the end of the workspace (the last region, 256-byte
    aligned, one row of H fp32 per (token, slot) and per shared token)."""

    shape = S.LayerShape(experts=16, hidden=1024, inter=512, topk=10, has_shared=shared)
    res, _ = layer(shape)
    t, k, h = 256, shape.topk, shape.hidden
    print(f"[experts] combine slot order k={k} shared={shared}", flush=True)
    x = S.make_hidden(t, h, seed=19, device=DEV)
    r = route_from_logits(S.make_logits(t, shape.experts, seed=20, device=DEV), topk=k)
    ids, weights = r.routing_ids, r.routing_weights
    bs = ops.block_size_m(t, k, shape.experts)
    align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=shape.experts)
    out = torch.empty((t, h), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.experts_workspace_bytes(t, k, h, shape.inter, shared), dtype=torch.uint8, device=DEV)
    ops.experts_w4a16_into(
        x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
        experts=shape.experts,
        inter=shape.inter, has_shared=shared, route_weights=weights,
        sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
        num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=0.0,
        out=out, workspace=ws)
    torch.cuda.synchronize()
    rows = t * k + (t if shared else 0)
    contrib = ws[ws.numel() - rows * h * 4:].view(torch.float32).view(rows, h)
    slots = contrib[: t * k].view(t, k, h)

    def in_order(order, shared_first=False):
        s = contrib[t * k:].clone() if shared and shared_first else None
        for j in order:
            s = slots[:, j].clone() if s is None else s + slots[:, j]
        if shared and not shared_first:
            s = s + contrib[t * k:]
        return s.to(torch.bfloat16).view(torch.int16)

    want = in_order(list(range(k)))
    assert torch.equal(out.view(torch.int16), want)
    # the check can tell orders apart: other orders round differently somewhere
    # (1 element in a few thousand straddles a bf16 rounding boundary)
    assert not torch.equal(want, in_order(list(range(k))[::-1]))
    if shared:
        assert not torch.equal(want, in_order(list(range(k)), shared_first=True))


@pytest.mark.parametrize("t", [1, 8, 64, 256])
def test_flash_decode(t):
    rows = np.unique(np.r_[np.arange(min(t, 6)), t - 1])
    check_layer(S.FLASH, t, rows=rows, seed=11 + t, clamp=10.0)


def test_flash_prefill_2048_subset():
    check_layer(S.FLASH, 2048, rows=[0, 1, 777, 2047], seed=13)


def test_flash_zipf_routing_subset():
    ids = S.zipf_ids(512, 256, 6, device=DEV)
    check_layer(S.FLASH, 512, rows=[0, 5, 511], seed=15, ids=ids)


def test_flash_prefill_8192_zipf_subset():
    """Zipf(1.1) routing at T=8192: the hottest experts span dozens of
    alignment blocks (many 128-slot chunks), cold experts a partial block."""
    ids = S.zipf_ids(8192, 256, 6, device=DEV)
    counts = torch.bincount(ids.flatten(), minlength=256)
    hot = int(torch.argmax(counts))
    hot_rows = torch.nonzero((ids == hot).any(dim=1)).flatten()[[0, -1]].cpu().numpy()
    check_layer(S.FLASH, 8192, rows=np.r_[0, 4097, 8191, hot_rows], seed=17, ids=ids)


def _custom_layer_check(shape, s13_fn, s2_fn, ts, seed):
    w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=seed, device=DEV)
    g = torch.Generator(DEV).manual_seed(seed)
    s13 = s13_fn(s13, g)
    s2 = s2_fn(s2, g)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts,
                                                        has_shared=shape.has_shared)
    src = DeviceExpertSource(w13, s13, w2, s2)
    for t in ts:
        x = S.make_hidden(t, shape.hidden, seed=seed + t, device=DEV)
        r = route_from_logits(S.make_logits(t, shape.experts, seed=seed + t + 1, device=DEV), topk=shape.topk)
        bs = ops.block_size_m(t, shape.topk, shape.experts)
        align = deterministic_moe_align_block_size(r.routing_ids, block_size=bs, num_experts=shape.experts)
        out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(ops.experts_workspace_bytes(t, shape.topk, shape.hidden, shape.inter, shape.has_shared),
                         dtype=torch.uint8, device=DEV)
        ops.experts_w4a16_into(
            x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
        experts=shape.experts,
            inter=shape.inter, has_shared=shape.has_shared, route_weights=r.routing_weights,
            sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
            num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=0.0,
            out=out, workspace=ws)
        torch.cuda.synchronize()
        ref = O.moe_fp32(to_np_f32(x), r.routing_ids.cpu().numpy(), r.routing_weights.cpu().numpy(), src,
                         shared_index=shape.experts if shape.has_shared else None)
        err = assert_moe_close(to_np_f32(out), ref, what=f"T={t} bs={bs}")
        print(f"    T={t} bs={bs} {err}", flush=True)


def test_zero_scale_groups_decode_and_prefill():
    """Groups with zero scales (and whole zero rows) contribute nothing; the
    packer's canonical form keeps the prefill scale ratios finite."""
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)

    def zero_some(s, g):
        mask = torch.rand(s.shape, device=DEV, generator=g) < 0.25
        s = torch.where(mask, torch.zeros_like(s), s)
        s[:, 3, :] = 0.0
        return s

    _custom_layer_check(shape, zero_some, zero_some, ts=(8, 64, 200), seed=21)


def test_wide_scale_range_prefill():
    """Scales spanning 2^-14 .. 2^6 within a row: the running sum is kept
    divided by the current group's scale, so consecutive ratios reach 2^20."""
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)

    def wide(s, g):
        e = torch.randint(-14, 7, s.shape, device=DEV, generator=g).float()
        return (torch.exp2(e) * (1.0 + torch.rand(s.shape, device=DEV, generator=g))).to(torch.bfloat16)

    _custom_layer_check(shape, wide, wide, ts=(64, 200), seed=23)


def test_extreme_scale_spread_takes_the_exact_path():
    """An expert whose gate rows put a 2^100 group scale next to a 2^-100 one
    (the running-sum ratio alone would be 2^200, beyond fp32) is marked by
    the ratio packer -- exactly the experts the oracle's rule names -- and its
    prefill blocks go through the exact-scaling kernel: the prefill output
    (blocks of 64) equals the decode kernels' (blocks of 16, exact per-group
    scaling) and the fp32 oracle, on every row, while the other experts keep
    the running-sum path."""

    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    print("[experts] extreme scale spread", flush=True)
    w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=31, device=DEV)
    # expert 3: gate rows [0, I) alternate 2^100 / 2^-100 per group; the up rows
    # stay ordinary, so h and the outputs stay within fp32
    g = torch.arange(s13.shape[-1], device=DEV)
    wild = torch.where(g % 2 == 0, torch.tensor(2.0 ** 100, device=DEV), torch.tensor(2.0 ** -100, device=DEV))
    s13[3, :shape.inter] = (wild * 1e-2).to(torch.bfloat16)
    # expert 5: a spread of 2^40 only, below the bound: stays on the fast path
    s2[5] = (s2[5].float() * torch.where(torch.arange(s2.shape[-1], device=DEV) % 2 == 0, 2.0 ** 20,
                                        2.0 ** -20)).to(torch.bfloat16)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts, has_shared=True)
    torch.cuda.synchronize()
    marked13 = (res.w13_r[:, 0] != 0).cpu().numpy()
    marked2 = (res.w2_r[:, 0] != 0).cpu().numpy()
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(marked13, O.needs_exact_scaling(bits(s13)))
    np.testing.assert_array_equal(marked2, O.needs_exact_scaling(bits(s2)))
    assert marked13.tolist() == [False, False, False, True, False, False, False, False, False]
    assert not marked2.any()
    # the stack-level mark (element 1 of the first expert's ratios)
    assert float(res.w13_r[0, 1]) == 1.0 and float(res.w2_r[0, 1]) == 0.0
    src = DeviceExpertSource(w13, s13, w2, s2)
    t = 256
    x = S.make_hidden(t, shape.hidden, seed=32, device=DEV)
    ids = torch.stack([torch.full((t,), 3, device=DEV), (torch.arange(t, device=DEV) % 7 + 4) % 8], dim=1)
    ids[::5, 1] = 5
    ids = ids.to(torch.int32)
    w = torch.full((t, 2), 0.5, device=DEV, dtype=torch.float32)
    outs = {}
    for bs in (16, 64):
        align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=shape.experts)
        out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(ops.experts_workspace_bytes(t, 2, shape.hidden, shape.inter, True), dtype=torch.uint8,
                         device=DEV)
        ops.experts_w4a16_into(
            x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
            experts=shape.experts, inter=shape.inter, has_shared=True, route_weights=w,
            sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
            num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=0.0, out=out,
            workspace=ws)
        torch.cuda.synchronize()
        outs[bs] = to_np_f32(out)
        assert np.isfinite(outs[bs]).all(), bs
    ref = O.moe_fp32(to_np_f32(x), ids.cpu().numpy(), w.cpu().numpy(), src, shared_index=shape.experts)
    assert np.abs(ref).max() > 1e25  # the 2^100 groups dominate
    assert_moe_close(outs[64], outs[16], what="prefill (exact path) vs decode")
    assert_moe_close(outs[64], ref, what="prefill (exact path) vs oracle")
    assert_moe_close(outs[16], ref, what="decode vs oracle")


@pytest.mark.parametrize("t,zipf", [(40, False), (600, False), (300, True)])
def test_paired_8_slot_blocks_equal_16_slot_blocks(t, zipf):
    """Decode blocks of 8 slots pair up (two consecutive blocks of one expert
    taken as one 16-slot item) once the experts average at least 4 slots per
    block: the output equals, bit for bit, the same routing aligned in blocks
    of 16 (a slot's result does not depend on how slots are grouped),
    including runs longer than the 16-block position scan (T=600: about 19
    blocks per expert) and Zipf routing, and matches the fp32 oracle."""

    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    print(f"[experts] paired 8-slot blocks T={t} zipf={zipf}", flush=True)
    x = S.make_hidden(t, shape.hidden, seed=61, device=DEV)
    r = route_from_logits(S.make_logits(t, shape.experts, seed=62, device=DEV), topk=shape.topk)
    ids = S.zipf_ids(t, shape.experts, shape.topk, seed=63, device=DEV) if zipf else r.routing_ids
    out8 = run_experts(shape, x, ids, r.routing_weights, block_size=8)
    out16 = run_experts(shape, x, ids, r.routing_weights, block_size=16)
    assert torch.equal(out8, out16)
    _, src = layer(shape)
    rows = np.arange(t) if t <= 64 else np.sort(np.random.default_rng(t).choice(t, 64, replace=False))
    ref = O.moe_fp32(to_np_f32(x), ids.cpu().numpy(), r.routing_weights.cpu().numpy(), src,
                     shared_index=shape.experts, rows=rows)
    assert_moe_close(to_np_f32(out8)[rows], ref, what=f"paired T={t}")
