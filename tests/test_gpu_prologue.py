"""The fused layer entry point (``dsv4moe_layer_w4a16``), whose prologue launch
aligns the route ids and sums the activation rows in one launch, and for
T <= 16 also routes (one workgroup routes every token and aligns the ids it
wrote; the others sum the activation rows); from 8192 route ids on, the
alignment is split over workgroups (chunk counts beside the row sums, then
chunk scatters).  Token counts on both sides of both thresholds, three score
functions, 8 / 256 / 1024 experts.

Checked bit for bit against the oracle's router (``model.py:564-584``,
``moe_forward.py:80-87``) and closed-form alignment
(``deterministic_moe_align.py:93-133``), and the layer output against the
staged launches (route, align, experts as separate entry points), which must
agree exactly because the row sums are summed in the same order.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import ResidentInt4MoEWeights, ops, synthetic as S

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SCORES = {"sigmoid": O.SCORE_SIGMOID, "softmax": O.SCORE_SOFTMAX, "sqrtsoftplus": O.SCORE_SQRTSOFTPLUS}
_CACHE: dict = {}


def resident(shape):
    key = (shape.experts, shape.hidden, shape.inter)
    if key not in _CACHE:
        w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=5, device=DEV)
        _CACHE[key] = ResidentInt4MoEWeights.from_checkpoint_layout(
            w13, s13, w2, s2, experts=shape.experts, has_shared=True)
    return _CACHE[key]


def run_layer(shape, tokens, score, seed, route_scale=1.5, clamp=0.0):
    res = resident(shape)
    E, H, I, k = shape.experts, shape.hidden, shape.inter, shape.topk
    g = torch.Generator(DEV).manual_seed(seed)
    x = S.make_hidden(tokens, H, seed=seed, device=DEV)
    logits = torch.randn((tokens, E), device=DEV, generator=g)
    bias = torch.randn((E,), device=DEV, generator=g) * 0.05 if score != "softmax" else None
    bs = ops.block_size_m(tokens, k, E)
    cap = O.max_padded_tokens(tokens * k, E, bs)
    nblocks = (cap + bs - 1) // bs
    ws = torch.empty(ops.experts_workspace_bytes(tokens, k, H, I, True), dtype=torch.uint8, device=DEV)

    def bufs():
        return dict(
            ids=torch.full((tokens, k), -7, dtype=torch.int32, device=DEV),
            weights=torch.full((tokens, k), -7.0, dtype=torch.float32, device=DEV),
            margin=torch.full((tokens,), -7.0, dtype=torch.float32, device=DEV),
            sorted=torch.full((cap,), -7, dtype=torch.int32, device=DEV),
            expert_ids=torch.full((nblocks,), -7, dtype=torch.int32, device=DEV),
            ntpp=torch.full((1,), -7, dtype=torch.int32, device=DEV),
            out=torch.empty((tokens, H), dtype=torch.bfloat16, device=DEV),
        )

    common = dict(w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
                  experts=E, inter=I,
                  has_shared=True, clamp_limit=clamp, block_size=bs)
    f = bufs()
    ops.layer_w4a16_into(x, logits, bias, topk=k, score_func=score, route_scale=route_scale, ids=f["ids"],
                         weights=f["weights"], margin=f["margin"], sorted_token_ids=f["sorted"],
                         expert_ids=f["expert_ids"], num_tokens_post_padded=f["ntpp"], out=f["out"],
                         workspace=ws, **common)
    st = bufs()
    ops.route_topk_into(logits, bias, topk=k, score_func=score, route_scale=route_scale, ids=st["ids"],
                        weights=st["weights"], margin=st["margin"])
    ops.align_into(st["ids"], block_size=bs, num_experts=E, sorted_token_ids=st["sorted"],
                   expert_ids=st["expert_ids"], num_tokens_post_padded=st["ntpp"])
    ops.experts_w4a16_into(x, route_weights=st["weights"], sorted_token_ids=st["sorted"],
                           expert_ids=st["expert_ids"], num_tokens_post_padded=st["ntpp"], out=st["out"],
                           workspace=ws, **common)
    torch.cuda.synchronize()
    ref = O.route_topk(logits.cpu().numpy(), k, score_func=SCORES[score],
                       bias=None if bias is None else bias.cpu().numpy(), route_scale=route_scale)
    al = O.moe_align(ref.ids, bs, E)
    return f, st, ref, al


def check(f, st, ref, al):
    np.testing.assert_array_equal(f["ids"].cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(f["weights"].cpu().numpy().view(np.uint32), ref.weights.view(np.uint32))
    np.testing.assert_array_equal(f["margin"].cpu().numpy().view(np.uint32), ref.margin.view(np.uint32))
    np.testing.assert_array_equal(f["sorted"].cpu().numpy(), al.sorted_token_ids)
    np.testing.assert_array_equal(f["expert_ids"].cpu().numpy(), al.expert_ids)
    assert int(f["ntpp"].item()) == al.num_tokens_post_padded
    assert torch.equal(f["out"], st["out"])


@pytest.mark.parametrize("score", list(SCORES))
@pytest.mark.parametrize("tokens", [1, 5, 16, 17, 64, 130])
def test_layer_entry_small_layer(score, tokens):
    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    print(f"[prologue] E=8 k=2 T={tokens} {score}", flush=True)
    check(*run_layer(shape, tokens, score, seed=100 + tokens))


@pytest.mark.parametrize("tokens", [1, 8, 10, 11, 17, 64, 96])
def test_layer_entry_256_experts(tokens):
    shape = S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True)
    print(f"[prologue] E=256 k=6 T={tokens}", flush=True)
    check(*run_layer(shape, tokens, "sqrtsoftplus", seed=200 + tokens, route_scale=2.5, clamp=10.0))


@pytest.mark.parametrize("tokens", [1, 3, 16, 64])
def test_layer_entry_1024_experts(tokens):
    shape = S.LayerShape(experts=1024, hidden=512, inter=512, topk=8, has_shared=True)
    print(f"[prologue] E=1024 k=8 T={tokens}", flush=True)
    check(*run_layer(shape, tokens, "sigmoid", seed=300 + tokens))


@pytest.mark.parametrize("shape,tokens", [
    (S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True), 1366),
    (S.LayerShape(experts=256, hidden=512, inter=512, topk=6, has_shared=True), 3000),
    (S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True), 4096),
])
def test_layer_entry_split_alignment(shape, tokens):
    """tokens * topk >= 8192: the layer aligns with the two-launch split (row
    sums beside the chunk counts, scratch in the workspace's contribution
    region); the staged chain aligns in one workgroup.  Same bits."""

    print(f"[prologue] split align E={shape.experts} k={shape.topk} T={tokens}", flush=True)
    check(*run_layer(shape, tokens, "sqrtsoftplus", seed=400 + tokens, route_scale=2.5, clamp=10.0))


@pytest.mark.parametrize("nan_cols", [[3], list(range(8))])
def test_layer_entry_one_token_nan_logits_matches_staged(nan_cols):
    """One routed token aligns in closed form when its k ids are distinct and
    in range; logits with NaN entries may give the router other ids, and
    whatever they are, the fused call must write exactly what the staged
    route + align + experts launches write (the closed form, or align_block
    when the ids repeat or leave the expert range)."""

    shape = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
    res = resident(shape)
    E, H, I, k = shape.experts, shape.hidden, shape.inter, shape.topk
    x = S.make_hidden(1, H, seed=7, device=DEV)
    logits = torch.randn((1, E), device=DEV, generator=torch.Generator(DEV).manual_seed(8))
    logits[0, nan_cols] = float("nan")
    bs = ops.block_size_m(1, k, E)
    cap = O.max_padded_tokens(k, E, bs)
    nblocks = (cap + bs - 1) // bs
    ws = torch.empty(ops.experts_workspace_bytes(1, k, H, I, True), dtype=torch.uint8, device=DEV)

    def bufs():
        return dict(ids=torch.full((1, k), -7, dtype=torch.int32, device=DEV),
                    weights=torch.full((1, k), -7.0, dtype=torch.float32, device=DEV),
                    sorted=torch.full((cap,), -7, dtype=torch.int32, device=DEV),
                    expert_ids=torch.full((nblocks,), -7, dtype=torch.int32, device=DEV),
                    ntpp=torch.full((1,), -7, dtype=torch.int32, device=DEV))

    print(f"[prologue] T=1 NaN logits at {nan_cols}", flush=True)
    f, st = bufs(), bufs()
    out_f = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    out_s = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    common = dict(w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, w13r=res.w13_r, w2r=res.w2_r,
                  experts=E, inter=I, has_shared=True, clamp_limit=0.0, block_size=bs)
    ops.layer_w4a16_into(x, logits, None, topk=k, score_func="sigmoid", route_scale=1.0, ids=f["ids"],
                         weights=f["weights"], margin=None, sorted_token_ids=f["sorted"],
                         expert_ids=f["expert_ids"], num_tokens_post_padded=f["ntpp"], out=out_f,
                         workspace=ws, **common)
    ops.route_topk_into(logits, None, topk=k, score_func="sigmoid", route_scale=1.0, ids=st["ids"],
                        weights=st["weights"], margin=None)
    ops.align_into(st["ids"], block_size=bs, num_experts=E, sorted_token_ids=st["sorted"],
                   expert_ids=st["expert_ids"], num_tokens_post_padded=st["ntpp"])
    ops.experts_w4a16_into(x, route_weights=st["weights"], sorted_token_ids=st["sorted"],
                           expert_ids=st["expert_ids"], num_tokens_post_padded=st["ntpp"], out=out_s,
                           workspace=ws, **common)
    torch.cuda.synchronize()
    for name in ("ids", "sorted", "expert_ids", "ntpp"):
        assert torch.equal(f[name], st[name]), name
    assert torch.equal(f["weights"].view(torch.int32), st["weights"].view(torch.int32))
    assert torch.equal(out_f.view(torch.int16), out_s.view(torch.int16))
