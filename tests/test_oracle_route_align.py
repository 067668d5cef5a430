"""Pins the oracle's router and alignment.

Router: brute force with Python's sorted() on an explicit key, torch's
sigmoid + topk on rows without near-ties, and the route invariants of
runtime/dsv4_direct/moe_runtime.py:463-475 and e0cf_tp4_moe_forward.py:497-527.
Alignment: the list brute force of fixed_moe_align.py:434-456 (restated as
moe_align_bruteforce), the known answers of the block-size policy and
capacity, and the layout invariants.
"""

import numpy as np
import pytest
import torch

import oracle as O


@pytest.mark.parametrize("score", [O.SCORE_SIGMOID, O.SCORE_SOFTMAX, O.SCORE_SQRTSOFTPLUS])
def test_route_bruteforce_small(score):
    rng = np.random.default_rng(10 + score)
    for trial in range(30):
        t, e = int(rng.integers(1, 6)), int(rng.integers(2, 20))
        k = int(rng.integers(1, e + 1))
        logits = rng.integers(-3, 4, size=(t, e)).astype(np.float32)  # many exact ties
        bias = rng.integers(-1, 2, size=e).astype(np.float32) * 0.25 if trial % 2 else None
        r = O.route_topk(logits, k, score_func=score, bias=bias, route_scale=1.5)
        scores = O.route_scores(logits, score)
        for i in range(t):
            sel = [float(scores[i, j]) + (0.0 if bias is None else float(bias[j])) for j in range(e)]
            sel32 = [np.float32(v) for v in (scores[i] + (0 if bias is None else bias)).astype(np.float32)]
            order = sorted(range(e), key=lambda j: (-sel32[j], j))
            assert list(r.ids[i]) == order[:k]
            if k < e:
                assert r.margin[i] == np.float32(sel32[order[k - 1]] - sel32[order[k]])
            w = [scores[i, j] for j in order[:k]]
            if score != O.SCORE_SOFTMAX:
                tot = np.float32(w[0])
                for v in w[1:]:
                    tot = np.float32(tot + v)
                w = [np.float32(v / tot) for v in w]
            np.testing.assert_array_equal(r.weights[i], np.float32(1.5) * np.asarray(w, dtype=np.float32))
            del sel


def test_route_agrees_with_torch_off_ties():
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((2048, 256)).astype(np.float32)
    r = O.route_topk(logits, 6, score_func=O.SCORE_SIGMOID)
    s = torch.from_numpy(logits).sigmoid()
    vals, ids = s.topk(7, dim=-1)
    safe = (vals[:, 5] - vals[:, 6]).numpy() > 4e-7
    assert safe.mean() > 0.99
    np.testing.assert_array_equal(r.ids[safe], ids[:, :6].numpy()[safe])
    r2 = O.route_topk(logits, 6, score_func=O.SCORE_SQRTSOFTPLUS, route_scale=1.5)
    s2 = torch.nn.functional.softplus(torch.from_numpy(logits)).sqrt()
    v2, i2 = s2.topk(7, dim=-1)
    safe2 = (v2[:, 5] - v2[:, 6]).numpy() > 4e-7
    np.testing.assert_array_equal(r2.ids[safe2], i2[:, :6].numpy()[safe2])


@pytest.mark.parametrize("score", [O.SCORE_SIGMOID, O.SCORE_SQRTSOFTPLUS])
def test_route_invariants(score):
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((4096, 256)).astype(np.float32)
    r = O.route_topk(logits, 6, score_func=score, bias=(rng.standard_normal(256) * 0.1).astype(np.float32),
                     route_scale=1.5)
    assert r.ids.min() >= 0 and r.ids.max() < 256
    s = np.sort(r.ids, axis=1)
    assert not (s[:, 1:] == s[:, :-1]).any()
    tol = 8 * np.finfo(np.float32).eps * 1.5
    assert np.abs(r.weights.astype(np.float64).sum(1) - 1.5).max() <= tol
    assert (r.margin >= 0).all()
    assert (r.weights > 0).all()


def test_softmax_weights_not_renormalised():
    rng = np.random.default_rng(13)
    logits = rng.standard_normal((16, 8)).astype(np.float32)
    r = O.route_topk(logits, 2, score_func=O.SCORE_SOFTMAX, route_scale=2.0)
    sm = O.softmax_f32(logits)
    np.testing.assert_array_equal(r.weights, np.take_along_axis(sm, r.ids, 1) * np.float32(2.0))


def test_hash_route_closed_form():
    rng = np.random.default_rng(14)
    logits = rng.standard_normal((20, 16)).astype(np.float32)
    table = np.stack([rng.permutation(16)[:3] for _ in range(50)]).astype(np.int64)
    toks = rng.integers(0, 50, size=20)
    r = O.hash_route(logits, table, toks, route_scale=1.5)
    np.testing.assert_array_equal(r.ids, table[toks])
    sc = O.sqrtsoftplus_f32(logits)
    for i in range(20):
        w = sc[i, table[toks[i]]]
        tot = np.float32(np.float32(w[0] + w[1]) + w[2])
        np.testing.assert_array_equal(r.weights[i], (w / tot).astype(np.float32) * np.float32(1.5))


def test_block_size_and_capacity_known_answers():
    # e0cf-moe-titan064.log:54-56 -- T=4 rows, k=6, E=256 -> block 8, capacity 192
    assert O.marlin_block_size_m(4, 6, 256) == 8
    assert O.max_padded_tokens(4 * 6, 256, 8) == 192
    # fixed_moe_align.py:29-38 -- [240,6], E=256, block 8 -> 3232 rows, 404 blocks
    cap = O.max_padded_tokens(240 * 6, 256, 8)
    assert cap == 3232 and cap // 8 == 404
    # policy thresholds (moe_runtime.py:291-300)
    assert O.marlin_block_size_m(64, 6, 256) == 8
    assert O.marlin_block_size_m(512, 6, 256) == 16
    assert O.marlin_block_size_m(1024, 6, 256) == 32
    assert O.marlin_block_size_m(2048, 6, 256) == 64
    assert O.marlin_block_size_m(8192, 6, 256) == 64
    assert O.marlin_block_size_m(4, 6, 256, act_itemsize=1) == 16
    assert O.max_padded_tokens(8192 * 6, 256, 64) == 65280
    with pytest.raises(ValueError):
        O.max_padded_tokens(0, 256, 8)


def _cases():
    rng = np.random.default_rng(15)
    out = []
    for _ in range(60):
        e = int(rng.integers(1, 40))
        t = int(rng.integers(1, 30))
        k = int(rng.integers(1, min(e, 6) + 1))
        ids = np.argsort(rng.random((t, e)), axis=1)[:, :k]
        out.append((ids, int(rng.choice([1, 2, 3, 8, 16, 64])), e))
    out.append((np.zeros((5, 1), dtype=np.int64), 8, 1))
    out.append((np.tile(np.arange(6), (40, 1)), 8, 256))
    return out


@pytest.mark.parametrize("case", range(62))
def test_align_closed_form_equals_bruteforce(case):
    ids, bs, e = _cases()[case]
    a = O.moe_align(ids, bs, e)
    b = O.moe_align_bruteforce(ids, bs, e)
    assert a.num_tokens_post_padded == b.num_tokens_post_padded
    np.testing.assert_array_equal(a.sorted_token_ids, b.sorted_token_ids)
    np.testing.assert_array_equal(a.expert_ids, b.expert_ids)


def test_align_invariants_large():
    rng = np.random.default_rng(16)
    t, e, k, bs = 8192, 256, 6, 64
    ids = np.argsort(rng.random((t, e)), axis=1)[:, :k]
    a = O.moe_align(ids, bs, e)
    n = a.num_tokens_post_padded
    s = a.sorted_token_ids
    real = s[s < t * k]
    np.testing.assert_array_equal(np.sort(real), np.arange(t * k))  # multiset
    assert n % bs == 0 and (s[n:] == t * k).all()
    flat = ids.reshape(-1)
    blocks = a.expert_ids
    active = blocks[: n // bs]
    assert (np.diff(active) >= 0).all() and (blocks[n // bs:] == -1).all()
    for b in range(n // bs):
        run = s[b * bs:(b + 1) * bs]
        vals = run[run < t * k]
        assert (flat[vals] == active[b]).all()
        assert (np.diff(vals) > 0).all()  # ascending within each run
