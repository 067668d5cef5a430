"""The grouped expert kernels read the alignment (padded count, block expert
ids, sorted slot ids) from device memory that a caller -- or a caller's
alignment provider -- writes, so they never use it to address memory without
a bound:

* a padded count above the capacity runs only the blocks that lie inside the
  sorted-id buffer (the result equals the valid alignment's);
* a block whose expert id is outside [0, experts) reads expert 0's weights
  (in bounds) and turns its slots' contributions into NaN, so the tokens it
  touched come out NaN and every other token is unchanged;
* a negative padded count (the alignment kernel's report of a route id out
  of range) makes the combine write NaN for every token.

Regression tests of the fixed kernels (decode and prefill block sizes, the
W4A16, W4A8 and MXFP4 paths); every launch stays in bounds.
"""

import pytest
import torch

from gaiban_lite_amd import (
    ResidentInt4MoEWeights,
    ResidentMXFP4MoEWeights,
    ops,
    route_from_logits,
    synthetic as S,
)
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SHAPE = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
_RES: dict = {}


def resident(fmt):
    if fmt not in _RES:
        if fmt == "mxfp4":
            w = S.make_checkpoint_experts_mxfp4(SHAPE, seed=12, device=DEV)
            _RES[fmt] = ResidentMXFP4MoEWeights.from_checkpoint_layout(*w, experts=SHAPE.experts, has_shared=True)
        else:
            w = S.make_checkpoint_experts(SHAPE, seed=12, device=DEV)
            _RES[fmt] = ResidentInt4MoEWeights.from_checkpoint_layout(
                *w, experts=SHAPE.experts, has_shared=True,
                marlin_input_dtype=torch.float8_e4m3fn if fmt == "w4a8" else None)
    return _RES[fmt]


def run(fmt, x, weights, align, bs):
    res = resident(fmt)
    t = x.shape[0]
    k = weights.shape[1]
    ws_fn = ops.experts_w4a8_workspace_bytes if fmt == "w4a8" else ops.experts_workspace_bytes
    ws = torch.empty(ws_fn(t, k, SHAPE.hidden, SHAPE.inter, True), dtype=torch.uint8, device=DEV)
    out = torch.empty((t, SHAPE.hidden), dtype=torch.bfloat16, device=DEV)
    fn = {"w4a16": ops.experts_w4a16_into, "w4a8": ops.experts_w4a8_into, "mxfp4": ops.experts_mxfp4_into}[fmt]
    ratios = dict(w13r=res.w13_r, w2r=res.w2_r) if fmt == "w4a16" else {}
    fn(x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, **ratios, experts=SHAPE.experts,
       inter=SHAPE.inter,
       has_shared=True, route_weights=weights, sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
       num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=0.0, out=out, workspace=ws)
    torch.cuda.synchronize()
    return out


def clone_alignment(a):
    return type(a)(sorted_token_ids=a.sorted_token_ids.clone(), expert_ids=a.expert_ids.clone(),
                   num_tokens_post_padded=a.num_tokens_post_padded.clone())


@pytest.mark.parametrize("fmt", ["w4a16", "w4a8", "mxfp4"])
@pytest.mark.parametrize("t", [8, 64])  # block size 8 (decode kernels) and 32 (prefill kernels)
def test_corrupted_alignment_stays_in_bounds_and_shows(fmt, t):
    print(f"[guard] fmt={fmt} T={t}", flush=True)
    x = S.make_hidden(t, SHAPE.hidden, seed=50 + t, device=DEV)
    r = route_from_logits(S.make_logits(t, SHAPE.experts, seed=51 + t, device=DEV), topk=SHAPE.topk)
    bs = ops.block_size_m(t, SHAPE.topk, SHAPE.experts, 1 if fmt == "w4a8" else 2)
    good = deterministic_moe_align_block_size(r.routing_ids, block_size=bs, num_experts=SHAPE.experts)
    base = run(fmt, x, r.routing_weights, good, bs)
    assert torch.isfinite(base.float()).all()
    cap = good.sorted_token_ids.numel()
    ntpp = int(good.num_tokens_post_padded.item())

    # padded count far above the capacity: only the blocks inside the buffer run
    big = clone_alignment(good)
    big.num_tokens_post_padded.fill_(cap + 7 * bs)
    assert torch.equal(run(fmt, x, r.routing_weights, big, bs), base)

    # one active block names expert 1000 (and another -5): its tokens turn NaN
    bad = clone_alignment(good)
    blocks = ntpp // bs
    hit = {0: 1000, blocks - 1: -5}
    touched = set()
    sorted_ids = good.sorted_token_ids.cpu()
    for blk, eid in hit.items():
        bad.expert_ids[blk] = eid
        for f in sorted_ids[blk * bs:(blk + 1) * bs].tolist():
            if f < t * SHAPE.topk:
                touched.add(f // SHAPE.topk)
    out = run(fmt, x, r.routing_weights, bad, bs)
    rows = torch.tensor(sorted(touched), device=DEV)
    others = torch.tensor([i for i in range(t) if i not in touched], device=DEV, dtype=torch.long)
    assert touched and torch.isnan(out[rows].float()).all()
    if others.numel():
        assert torch.equal(out[others], base[others])

    # negative padded count: every output NaN
    neg = clone_alignment(good)
    neg.num_tokens_post_padded.fill_(-1)
    assert torch.isnan(run(fmt, x, r.routing_weights, neg, bs).float()).all()


def test_out_of_range_route_id_makes_the_layer_output_nan():
    """A route id outside [0, experts) (e.g. from a corrupted provider) is
    reported by the alignment kernel as a negative padded count, and the
    experts call answers with an all-NaN output instead of stale values."""

    t, bs = 16, 8
    x = S.make_hidden(t, SHAPE.hidden, seed=70, device=DEV)
    r = route_from_logits(S.make_logits(t, SHAPE.experts, seed=71, device=DEV), topk=SHAPE.topk)
    ids = r.routing_ids.clone()
    ids[3, 1] = SHAPE.experts + 2
    align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=SHAPE.experts)
    assert int(align.num_tokens_post_padded.item()) == -1
    assert torch.isnan(run("w4a16", x, r.routing_weights, align, bs).float()).all()
