"""Pins of the oracle's parity metrics and hash router, and of the product's
``moe_forward.error_metrics`` (row a14 of the hot path).

* ``O.rel_fro`` (``runtime/c2f_dense_moe_gate.py:66-69``: ``||other -
  reference|| / ||reference||``) and ``O.error_metrics`` /
  ``moe_forward.error_metrics`` (``runtime/dsv4_direct/moe_forward.py:234-268``)
  against answers computed by hand: an asymmetric pair fixes which argument
  is the reference (a swapped denominator fails), a zero reference fixes the
  float32-eps floor of the denominator, and the non-finite, shape-mismatch
  and empty cases follow the reference's contract.
* ``O.hash_route`` against torch's own operations in the reference's order
  (``moe_forward.py:218-223``: ``F.softplus(F.linear(x, W)).sqrt()``, then
  ``tid2eid.index_select``, ``gather``, ``sum``, divide, ``* route_scale``),
  on seeded Flash-shape logits and random tables: ids equal, weights within
  8 ulp -- the bound the learned router is held to in
  ``test_oracle_torch_path.py``.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from gaiban_lite_amd import moe_forward as MF

EPS32 = float(np.finfo(np.float32).eps)


# --------------------------------------------------------------- rel_fro


def test_rel_fro_known_answers():
    # reference (0, 5), observed (3, 9): diff (3, 4), ||diff|| / ||reference|| = 5 / 5
    assert O.rel_fro([3.0, 9.0], [0.0, 5.0]) == pytest.approx(5.0 / 5.0, rel=1e-15)
    # asymmetric: the second argument is the reference (denominator)
    assert O.rel_fro([2.0, 0.0], [1.0, 0.0]) == pytest.approx(1.0, rel=1e-15)
    assert O.rel_fro([1.0, 0.0], [2.0, 0.0]) == pytest.approx(0.5, rel=1e-15)
    # sqrt(1 + 4 + 4) / sqrt(4 + 16 + 16 + 64) = 3 / 10
    assert O.rel_fro([[3.0, 2.0], [6.0, 8.0]], [[2.0, 4.0], [4.0, 8.0]]) == pytest.approx(0.3, rel=1e-15)
    assert O.rel_fro(np.ones(7), np.ones(7)) == 0.0


def test_rel_fro_is_scale_invariant_and_not_zero_for_a_difference():
    rng = np.random.default_rng(3)
    r = rng.standard_normal((64, 33)).astype(np.float32)
    o = r + 1e-3 * rng.standard_normal(r.shape).astype(np.float32)
    base = O.rel_fro(o, r)
    assert 5e-4 < base < 2e-3
    assert O.rel_fro(1024.0 * o, 1024.0 * r) == pytest.approx(base, rel=1e-12)
    # a planted all-zero observation is a 100% error, not a pass
    assert O.rel_fro(np.zeros_like(r), r) == pytest.approx(1.0, rel=1e-12)


# --------------------------------------------------------- error_metrics


def _metric_cases():
    # observed, reference, max_abs, rms_rel, reference_rms (by hand)
    return [
        # diff (0, 0, -2): rms sqrt(4/3); reference rms sqrt(30/3)
        ([1.0, 2.0, 3.0], [1.0, 2.0, 5.0], 2.0, math.sqrt(4.0 / 3.0) / math.sqrt(10.0), math.sqrt(10.0)),
        # identical
        ([[0.5, -1.5], [2.0, 4.0]], [[0.5, -1.5], [2.0, 4.0]], 0.0, 0.0, math.sqrt((0.25 + 2.25 + 4 + 16) / 4)),
        # asymmetric pair: reference (1, 1) -> rms 1; diff (3, -1) -> rms sqrt(5)
        ([4.0, 0.0], [1.0, 1.0], 3.0, math.sqrt(5.0), 1.0),
        ([1.0, 1.0], [4.0, 0.0], 3.0, math.sqrt(5.0) / math.sqrt(8.0), math.sqrt(8.0)),
        # zero reference: the denominator is float32 eps
        ([0.0, 0.0, 0.0, 1.0], [0.0, 0.0, 0.0, 0.0], 1.0, 0.5 / EPS32, 0.0),
    ]


@pytest.mark.parametrize("case", range(5))
def test_oracle_error_metrics_known_answers(case):
    o, r, max_abs, rms_rel, ref_rms = _metric_cases()[case]
    m = O.error_metrics(o, r)
    assert m["finite"] is True
    assert m["max_abs"] == pytest.approx(max_abs, rel=1e-12, abs=0.0)
    assert m["rms_rel"] == pytest.approx(rms_rel, rel=1e-12, abs=0.0)
    assert m["reference_rms"] == pytest.approx(ref_rms, rel=1e-12, abs=0.0)


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_product_error_metrics_known_answers(case, dtype):
    """The product metric takes tensors of any float dtype and compares in
    fp32, as the reference does (every case here is exact in bf16)."""

    o, r, max_abs, rms_rel, ref_rms = _metric_cases()[case]
    m = MF.error_metrics(torch.tensor(o, dtype=dtype), torch.tensor(r, dtype=dtype))
    assert set(m) == {"finite", "max_abs", "rms_rel", "reference_rms"}
    assert m["finite"] is True
    assert all(type(m[k]) is float for k in ("max_abs", "rms_rel", "reference_rms"))
    assert m["max_abs"] == pytest.approx(max_abs, rel=1e-6, abs=0.0)
    assert m["rms_rel"] == pytest.approx(rms_rel, rel=1e-6, abs=0.0)
    assert m["reference_rms"] == pytest.approx(ref_rms, rel=1e-6, abs=0.0)


@pytest.mark.parametrize("bad", [math.nan, math.inf, -math.inf])
@pytest.mark.parametrize("where", ["observed", "reference"])
def test_error_metrics_non_finite(bad, where):
    good = [1.0, 2.0, 3.0]
    poisoned = [1.0, bad, 3.0]
    o, r = (poisoned, good) if where == "observed" else (good, poisoned)
    want = {"finite": False, "max_abs": None, "rms_rel": None, "reference_rms": None}
    assert O.error_metrics(o, r) == want
    assert MF.error_metrics(torch.tensor(o), torch.tensor(r)) == want


def test_error_metrics_shape_and_empty_errors():
    with pytest.raises(ValueError):
        O.error_metrics(np.zeros((2, 3)), np.zeros((3, 2)))
    with pytest.raises(ValueError, match="empty"):
        O.error_metrics(np.zeros((0, 4)), np.zeros((0, 4)))
    with pytest.raises(ValueError, match="shape"):
        MF.error_metrics(torch.zeros(2, 3), torch.zeros(3, 2))
    with pytest.raises(ValueError, match="empty"):
        MF.error_metrics(torch.zeros(0, 4), torch.zeros(0, 4))
    # a broadcastable pair is still a shape mismatch
    with pytest.raises(ValueError):
        MF.error_metrics(torch.zeros(1, 4), torch.zeros(3, 4))


def test_product_and_oracle_metrics_agree_on_random_data():
    g = torch.Generator().manual_seed(21)
    r = torch.randn((256, 96), generator=g)
    o = r + 1e-2 * torch.randn((256, 96), generator=g)
    a = MF.error_metrics(o, r)
    b = O.error_metrics(o.numpy(), r.numpy())
    for k in ("max_abs", "rms_rel", "reference_rms"):
        assert a[k] == pytest.approx(b[k], rel=1e-5), k
    assert 5e-3 < a["rms_rel"] < 2e-2
    # the metric does not modify or require grad on its inputs
    o.requires_grad_(True)
    assert MF.error_metrics(o, r)["finite"] is True


# ------------------------------------------------------------- hash_route


def _ulp_f32(a, b):
    ia = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def _torch_hash_gate(logits, tid2eid, input_ids, route_scale):
    scores = F.softplus(logits.float()).sqrt()
    ids = tid2eid.index_select(0, input_ids)
    selected = scores.gather(1, ids)
    w = selected / selected.sum(dim=-1, keepdim=True)
    w = w * float(route_scale)
    return ids.to(torch.int32), w.float()


@pytest.mark.parametrize("tokens,route_scale,spread", [(64, 1.5, 1.0), (8192, 1.5, 1.0), (2048, 2.5, 8.0)])
def test_hash_route_against_torch_reference_ops(tokens, route_scale, spread):
    """Flash shape: 256 experts, top-6, a 129,280-entry token table.  The
    ``spread`` case scales the logits by 8 so that softplus crosses its
    threshold of 20 on some entries."""

    e, k, vocab = 256, 6, 129280
    g = torch.Generator().manual_seed(4000 + tokens)
    logits = torch.randn((tokens, e), generator=g) * spread
    tid2eid = torch.argsort(torch.rand((vocab, e), generator=g)[:, :64], dim=1)[:, :k].to(torch.int64)
    input_ids = torch.randint(0, vocab, (tokens,), generator=g, dtype=torch.int64)
    ref = O.hash_route(logits.numpy(), tid2eid.numpy(), input_ids.numpy(), route_scale=route_scale)
    tid, tw = _torch_hash_gate(logits, tid2eid, input_ids, route_scale)
    np.testing.assert_array_equal(ref.ids, tid.numpy())
    ulp = _ulp_f32(ref.weights, tw.numpy())
    assert ulp.max() <= 8, int(ulp.max())
    np.testing.assert_allclose(ref.weights.astype(np.float64).sum(1), route_scale,
                               rtol=8 * np.finfo(np.float32).eps)
    print(f"hash route T={tokens}: max weight ulp {int(ulp.max())}")


def test_hash_route_planted_mistakes_fail():
    """Planted mistakes in the oracle's hash router move the weights far
    outside the 8-ulp bound: a missing renormalisation, scores without the
    square root, and a dropped route scale."""

    g = torch.Generator().manual_seed(77)
    logits = torch.randn((128, 256), generator=g)
    tid2eid = torch.argsort(torch.rand((1000, 256), generator=g), dim=1)[:, :6].to(torch.int64)
    input_ids = torch.randint(0, 1000, (128,), generator=g, dtype=torch.int64)
    _, tw = _torch_hash_gate(logits, tid2eid, input_ids, 1.5)
    ids = tid2eid.numpy()[input_ids.numpy()]
    sc = O.sqrtsoftplus_f32(logits.numpy())
    sel = np.take_along_axis(sc, ids, 1)
    no_renorm = sel * np.float32(1.5)
    no_sqrt = np.take_along_axis(sc * sc, ids, 1)
    no_sqrt = no_sqrt / no_sqrt.sum(1, keepdims=True) * np.float32(1.5)
    no_scale = sel / sel.sum(1, keepdims=True)
    for wrong in (no_renorm, no_sqrt, no_scale):
        assert _ulp_f32(wrong.astype(np.float32), tw.numpy()).max() > 1000
