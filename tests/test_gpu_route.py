"""Router kernel parity: bit-exact ids, weights, margin and selection against the
CPU oracle (same fixed fp32 operation sequence), over every score function."""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import ops, route_from_logits

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SCORES = {"sigmoid": O.SCORE_SIGMOID, "softmax": O.SCORE_SOFTMAX, "sqrtsoftplus": O.SCORE_SQRTSOFTPLUS}


def run_gpu(logits_np, topk, score, bias_np=None, route_scale=1.0):
    t, e = logits_np.shape
    logits = torch.from_numpy(logits_np).to(DEV)
    bias = None if bias_np is None else torch.from_numpy(bias_np).to(DEV)
    depth = min(topk + 1, e)
    ids = torch.empty((t, topk), dtype=torch.int32, device=DEV)
    w = torch.empty((t, topk), dtype=torch.float32, device=DEV)
    margin = torch.empty((t,), dtype=torch.float32, device=DEV)
    sid = torch.empty((t, depth), dtype=torch.int32, device=DEV)
    ssc = torch.empty((t, depth), dtype=torch.float32, device=DEV)
    ops.route_topk_into(logits, bias, topk=topk, score_func=score, route_scale=route_scale,
                        ids=ids, weights=w, margin=margin, selection_ids=sid, selection_scores=ssc)
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (ids, w, margin, sid, ssc)]


def check_exact(logits_np, topk, score, bias_np=None, route_scale=1.0):
    ids, w, margin, sid, ssc = run_gpu(logits_np, topk, score, bias_np, route_scale)
    ref = O.route_topk(logits_np, topk, score_func=SCORES[score], bias=bias_np, route_scale=route_scale)
    np.testing.assert_array_equal(ids, ref.ids)
    np.testing.assert_array_equal(sid, ref.selection_ids)
    np.testing.assert_array_equal(w.view(np.uint32), ref.weights.view(np.uint32))
    np.testing.assert_array_equal(margin.view(np.uint32), ref.margin.view(np.uint32))
    np.testing.assert_array_equal(ssc.view(np.uint32), ref.selection_scores.view(np.uint32))


@pytest.mark.parametrize("score", list(SCORES))
@pytest.mark.parametrize("t,e,k", [(64, 8, 2), (1, 256, 6), (64, 256, 6), (8192, 256, 6),
                                   (37, 384, 8), (16, 1024, 16), (5, 130, 1), (3, 17, 16)])
def test_route_bit_exact(score, t, e, k):
    rng = np.random.default_rng(t * 7919 + e * 31 + k)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    check_exact(logits, k, score)


@pytest.mark.parametrize("score", list(SCORES))
def test_route_bias_and_scale(score):
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((256, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.05).astype(np.float32)
    check_exact(logits, 6, score, bias, route_scale=1.5)


@pytest.mark.parametrize("score", list(SCORES))
def test_route_ties_and_extremes(score):
    rng = np.random.default_rng(9)
    logits = rng.integers(-3, 4, size=(128, 256)).astype(np.float32)  # massive ties
    logits[0] = 0.0
    logits[1, :] = 25.0  # softplus threshold branch
    logits[2, :10] = -95.0  # exp underflow region
    logits[3, ::2] = 60.0
    check_exact(logits, 6, score)


def test_route_matches_torch_topk_off_ties():
    """Against torch's own sigmoid + topk: ids agree on every row whose top-k
    margin is not within a few ULPs (torch's sigmoid may differ by an ULP)."""

    rng = np.random.default_rng(11)
    logits = rng.standard_normal((4096, 256)).astype(np.float32)
    ids, w, margin, _, _ = run_gpu(logits, 6, "sigmoid")
    lt = torch.from_numpy(logits)
    scores = lt.sigmoid()
    vals, tids = scores.topk(7, dim=-1)
    safe = (vals[:, 5] - vals[:, 6]).numpy() > 4 * np.spacing(np.float32(1.0))
    assert safe.mean() > 0.99
    np.testing.assert_array_equal(ids[safe], tids[:, :6].numpy()[safe])
    tw = scores.gather(1, tids[:, :6])
    tw = (tw / tw.sum(-1, keepdim=True)).numpy()
    np.testing.assert_allclose(w[safe], tw[safe], rtol=5e-7, atol=0)


def test_route_from_logits_wrapper_invariants():
    logits = torch.randn(512, 256, device=DEV, generator=torch.Generator(DEV).manual_seed(3))
    r = route_from_logits(logits, topk=6, score_func="sqrtsoftplus", route_scale=1.5)
    ids = r.routing_ids.cpu()
    w = r.routing_weights.cpu()
    assert ids.dtype == torch.int32 and r.selection_ids.dtype == torch.int64
    assert int(ids.min()) >= 0 and int(ids.max()) < 256
    s = ids.sort(dim=1).values
    assert not bool((s[:, 1:] == s[:, :-1]).any())
    tol = 8 * torch.finfo(torch.float32).eps * 1.5
    assert float((w.sum(1) - 1.5).abs().max()) <= tol
    assert bool((r.margin.cpu() >= 0).all())


def test_route_hash_matches_oracle():
    rng = np.random.default_rng(13)
    t, e, k, vocab = 300, 256, 6, 1000
    logits = rng.standard_normal((t, e)).astype(np.float32)
    table = np.stack([rng.permutation(e)[:k] for _ in range(vocab)]).astype(np.int64)
    toks = rng.integers(0, vocab, size=t).astype(np.int64)
    ids = torch.empty((t, k), dtype=torch.int32, device=DEV)
    w = torch.empty((t, k), dtype=torch.float32, device=DEV)
    sel = torch.empty((t, k), dtype=torch.float32, device=DEV)
    ops.route_hash_into(torch.from_numpy(logits).to(DEV), torch.from_numpy(table).to(DEV),
                        torch.from_numpy(toks).to(DEV), route_scale=1.5, ids=ids, weights=w,
                        selected_scores=sel)
    ref = O.hash_route(logits, table, toks, route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), ref.weights.view(np.uint32))
    np.testing.assert_array_equal(sel.cpu().numpy().view(np.uint32),
                                  np.take_along_axis(ref.scores, ref.ids, 1).view(np.uint32))


@pytest.mark.parametrize("tokens,hidden,experts", [(1, 4096, 256), (100, 4096, 256), (1000, 4096, 256),
                                                    (8192, 4096, 256), (37, 1056, 72), (700, 1056, 256),
                                                    (600, 512, 200)])
def test_gate_logits_fp32_accumulation(tokens, hidden, experts):
    """Both gate kernels (K split over 8 wavefronts up to 512 tokens; 64 x 64
    LDS tiles above, when K is a multiple of 128) against a float64 product;
    ragged token / expert tiles and a K that splits unevenly; the same call
    twice gives the same bits."""

    print(f"[gate] T={tokens} H={hidden} E={experts}", flush=True)
    g = torch.Generator(DEV).manual_seed(21 + tokens)
    x = torch.randn(tokens, hidden, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(experts, hidden, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    logits = torch.full((tokens, experts), float("nan"), dtype=torch.float32, device=DEV)
    ops.gate_logits_into(x, wg, logits)
    again = torch.empty_like(logits)
    ops.gate_logits_into(x, wg, again)
    torch.cuda.synchronize()
    assert torch.equal(logits, again)
    ref = x.double().cpu() @ wg.double().cpu().T
    err = (logits.double().cpu() - ref).abs().max().item()
    assert err <= 1e-5 * ref.abs().max().item() + 1e-6, err
