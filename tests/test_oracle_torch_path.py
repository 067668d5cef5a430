"""The torch restatement of the reference's dense MoE path (``oracle/torch_path.py``)
and the numpy bf16 mirror (``oracle/moe_oracle.py:moe_bf16_mirror``), checked
against each other and against torch's own operations on the CPU.

* bf16 mode: the mirror emulates every bf16 cast of ``ops/dense_moe.py:336-354``
  and ``moe_runtime.py:246-263,1873`` in numpy; the restatement runs the same
  sequence with torch's bf16 ``matmul`` / ``F.linear`` / ``.to(bfloat16)``.
  The two differ only where fp32 accumulation order (or the last fp32 bit of
  SiLU) puts an intermediate one bf16 ulp apart, which then moves the outputs
  of that one row: at least 99.9% of the outputs must be bit-identical and
  every difference at most 2^-8 of the largest output.  Dropping any one of the mirror's bf16 casts
  (a planted mistake, monkeypatched into the oracle) must break that bar.
* fp32 mode: against ``moe_fp32`` to 1e-5 (both fp32, different summation
  order).
* dequantisers: bit-exact against the numpy oracle's.
* router: torch's sigmoid / sqrt-softplus -> topk(k+1) -> gather -> sum ->
  div (``moe_forward.py:80-87``) against the oracle's fixed-sequence router
  on seeded C2 / C3 logits, under stated ULP bounds, counting near-tie id
  differences.
"""

import numpy as np
import pytest
import torch

import oracle as O
from oracle import torch_path as TP

TINY_SHARED = dict(experts=8, hidden=1024, inter=512, topk=2)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _experts(e_total, hidden, inter, seed):
    g = torch.Generator().manual_seed(seed)
    w13 = torch.randint(0, 256, (e_total, 2 * inter, hidden // 2), dtype=torch.uint8, generator=g)
    s13 = (torch.rand((e_total, 2 * inter, hidden // 128), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    w2 = torch.randint(0, 256, (e_total, hidden, inter // 2), dtype=torch.uint8, generator=g)
    s2 = (torch.rand((e_total, hidden, inter // 128), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    return w13, s13, w2, s2


def _case(seed=0, t=64, clamp=0.0, shared=True):
    e, h, i, k = TINY_SHARED["experts"], TINY_SHARED["hidden"], TINY_SHARED["inter"], TINY_SHARED["topk"]
    w13, s13, w2, s2 = _experts(e + (1 if shared else 0), h, i, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn((t, h), generator=g).to(torch.bfloat16)
    logits = torch.randn((t, e), generator=g)
    r = O.route_topk(logits.numpy(), k, score_func=O.SCORE_SIGMOID)
    src = O.ExpertSource(w13.numpy(), _bits(s13), w2.numpy(), _bits(s2))
    stacked = TP.StackedExperts(w13, s13, w2, s2)
    return dict(x=x, ids=r.ids, weights=r.weights, src=src, stacked=stacked, e=e, shared=e if shared else None,
                clamp=clamp)


def _torch_bf16(c):
    return TP.dense_moe(c["x"], torch.from_numpy(c["ids"]), torch.from_numpy(c["weights"]), c["stacked"],
                        num_experts=c["e"], shared_index=c["shared"], clamp_limit=c["clamp"],
                        dtype=torch.bfloat16).float().numpy()


def _mirror(c):
    return O.moe_bf16_mirror(c["x"].float().numpy(), c["ids"], c["weights"], c["src"], shared_index=c["shared"],
                             clamp_limit=c["clamp"])


def _agreement(a, b):
    """(fraction of bit-identical outputs, max |a - b| / max |a|)."""
    ua = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    ub = np.ascontiguousarray(b, dtype=np.float32).view(np.uint32)
    same = float((ua == ub).mean())
    return same, float(np.abs(a - b).max() / max(np.abs(a).max(), 1e-30))


def test_dequant_int4_matches_numpy_oracle():
    w13, s13, _, _ = _experts(2, 256, 128, seed=3)
    got = TP.dequant_int4_g128(w13[1], s13[1]).numpy()
    want = O.dequant_int4_g128(w13[1].numpy(), _bits(s13[1]))
    assert np.array_equal(got, want)
    got16 = TP.dequant_int4_g128(w13[1], s13[1], dtype=torch.bfloat16).float().numpy()
    assert np.array_equal(got16, O.bf16_round(want))


def test_dequant_mxfp4_matches_numpy_oracle_every_code_and_scale():
    codes = torch.arange(256, dtype=torch.uint8).repeat(254, 1)  # every byte on every row
    scales = torch.arange(0, 254, dtype=torch.uint8).view(254, 1).repeat(1, 16)  # every valid E8M0 byte
    got = TP.dequant_mxfp4(codes, scales).numpy()
    want = O.dequant_mxfp4(codes.numpy(), scales.numpy())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        TP.decode_e8m0(torch.tensor([255], dtype=torch.uint8))


@pytest.mark.parametrize("clamp", [0.0, 10.0, 2.0])
def test_bf16_restatement_matches_mirror_bits(clamp):
    c = _case(seed=5, clamp=clamp)
    same, dev = _agreement(_torch_bf16(c), _mirror(c))
    assert same >= 0.999 and dev <= 2.0 ** -8, (same, dev)


def test_bf16_restatement_without_shared_expert():
    c = _case(seed=6, shared=False)
    same, dev = _agreement(_torch_bf16(c), _mirror(c))
    assert same >= 0.999 and dev <= 2.0 ** -8, (same, dev)


@pytest.mark.parametrize("dropped", sorted(O.BF16_CASTS.keys() - {"input"}))
def test_dropping_any_bf16_cast_breaks_bit_agreement(dropped, monkeypatch):
    """Planted mistake: one of the mirror's bf16 casts becomes the identity
    (``input`` is exact here: the inputs are bf16 already).  Measured: 38-81%
    of the outputs stay bit-identical, against 99.96% for the true order."""

    c = _case(seed=5)
    want = _torch_bf16(c)
    monkeypatch.setitem(O.BF16_CASTS, dropped, lambda v: np.asarray(v, dtype=np.float32))
    same, _ = _agreement(want, _mirror(c))
    assert same < 0.9, (dropped, same)


def test_fp32_restatement_matches_moe_fp32():
    c = _case(seed=9, clamp=10.0)
    got = TP.dense_moe(c["x"], torch.from_numpy(c["ids"]), torch.from_numpy(c["weights"]), c["stacked"],
                       num_experts=c["e"], shared_index=c["shared"], clamp_limit=10.0,
                       dtype=torch.float32).numpy()
    want = O.moe_fp32(c["x"].float().numpy(), c["ids"], c["weights"], c["src"], shared_index=c["shared"],
                      clamp_limit=10.0)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_moe_fp32_workers_equal_serial():
    c = _case(seed=11)
    a = O.moe_fp32(c["x"].float().numpy(), c["ids"], c["weights"], c["src"], shared_index=c["shared"])
    b = O.moe_fp32(c["x"].float().numpy(), c["ids"], c["weights"], c["src"], shared_index=c["shared"], workers=4)
    assert np.array_equal(a, b)


def _ulp_f32(a, b):
    ia = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("score,tokens", [("sigmoid", 256), ("sigmoid", 8192), ("sqrtsoftplus", 8192)])
def test_router_against_torch_reference_ops(score, tokens):
    """Weights and margin of the oracle router (the GPU router is bit-exact
    with it) against torch's own score / topk / gather / sum / div sequence.
    Bounds: ids may differ only where torch's and the oracle's scores order a
    near-tie differently (gap <= 4 ulp of the k-th score); on the other rows
    weights are within 8 ulp and the margin within 8 ulp of the k-th score."""

    e, k = 256, 6
    g = torch.Generator().manual_seed(1000 + tokens)
    logits = torch.randn((tokens, e), generator=g)
    bias = (torch.randn((e,), generator=g) * 0.05) if score == "sqrtsoftplus" else None
    code = O.SCORE_SIGMOID if score == "sigmoid" else O.SCORE_SQRTSOFTPLUS
    ref = O.route_topk(logits.numpy(), k, score_func=code, bias=None if bias is None else bias.numpy(),
                       route_scale=1.5)
    tid, tw, tm = TP.gate_route(logits, topk=k, score_func=score, bias=bias, route_scale=1.5)
    tid, tw, tm = tid.numpy(), tw.numpy(), tm.numpy()
    same_rows = (np.sort(tid, axis=1) == np.sort(ref.ids, axis=1)).all(axis=1)
    diff_rows = np.nonzero(~same_rows)[0]
    # every id difference is a near-tie in the oracle's own selection scores
    for r in diff_rows:
        sel = ref.selection_scores[r]
        gap = _ulp_f32(sel[k - 1], sel[k])
        assert gap <= 4, (r, sel[k - 1], sel[k])
    assert len(diff_rows) <= max(2, tokens // 1000), len(diff_rows)
    ok = np.nonzero(same_rows & (tid == ref.ids).all(axis=1))[0]
    assert len(ok) >= tokens - 2 * len(diff_rows) - tokens // 500
    assert _ulp_f32(tw[ok], ref.weights[ok]).max() <= 8
    kth = np.abs(ref.selection_scores[ok, k - 1])
    ulp_kth = np.spacing(kth.astype(np.float32))
    assert (np.abs(tm[ok] - ref.margin[ok]) <= 8 * ulp_kth).all()
    print(f"{score} T={tokens}: id-differing rows {len(diff_rows)}, max weight ulp "
          f"{int(_ulp_f32(tw[ok], ref.weights[ok]).max())}")
