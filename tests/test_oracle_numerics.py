"""Pins the oracle's elementary functions and rounding helpers.

The fixed fp32 operation sequences (shared by the HIP router) are checked
against float64 closed forms; bf16 / fp8 rounding against torch's own dtype
conversions; the combine rounding against the reference's exhaustive KAT
(bf16 add with fp32 opmath == fp32 add then one bf16 rounding,
runtime/c2f_moe_combine_gate.py:54-84) on a large sample.
"""

import numpy as np
import pytest
import torch

import oracle as O


def ulps(a, ref):
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    sp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(a - ref) / sp


def test_exp_accuracy_and_special_values():
    x = np.linspace(-86.5, 88.0, 400001).astype(np.float32)
    assert ulps(O.exp_f32(x), np.exp(x.astype(np.float64))).max() <= 2.0
    assert O.exp_f32(np.float32(0.0)) == 1.0
    # results whose binary exponent n = rint(x log2 e) <= -126 flush to 0
    assert O.exp_f32(np.float32(-87.0)) == 0.0  # n = rint(-125.51) = -126
    assert O.exp_f32(np.float32(-86.9)) > 0.0    # n = -125
    assert O.exp_f32(np.float32(-200.0)) == 0.0  # clamped, no subnormal results
    assert np.isinf(O.exp_f32(np.float32(200.0)))


def test_log_log1p_accuracy():
    w = np.exp(np.linspace(0.0, 21.0, 200001)).astype(np.float32)
    assert ulps(O.log_f32(w), np.log(w.astype(np.float64))).max() <= 2.0
    assert O.log_f32(np.float32(1.0)) == 0.0
    u = np.exp(np.linspace(-60.0, 6.0, 200001)).astype(np.float32)
    assert ulps(O.log1p_f32(u), np.log1p(u.astype(np.float64))).max() <= 4.0
    tiny = np.float32(1e-30)
    assert O.log1p_f32(tiny) == tiny  # 1 + u == 1 branch returns u exactly


def test_score_functions():
    x = np.linspace(-40.0, 40.0, 200001).astype(np.float32)
    x64 = x.astype(np.float64)
    assert ulps(O.sigmoid_f32(x), 1.0 / (1.0 + np.exp(-x64))).max() <= 3.0
    assert O.sigmoid_f32(np.float32(0.0)) == 0.5
    y = np.linspace(-15.0, 19.99, 200001).astype(np.float32)
    ref = np.sqrt(np.log1p(np.exp(y.astype(np.float64))))
    assert ulps(O.sqrtsoftplus_f32(y), ref).max() <= 4.0
    # torch softplus threshold: x > 20 returns x itself
    big = np.array([20.5, 50.0, 1e4], dtype=np.float32)
    np.testing.assert_array_equal(O.sqrtsoftplus_f32(big), np.sqrt(big))
    lg = np.random.default_rng(0).standard_normal((64, 256)).astype(np.float32) * 3
    sm = O.softmax_f32(lg)
    r = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    r /= r.sum(1, keepdims=True)
    assert ulps(sm, r).max() <= 32.0  # fp32 sum of 256 terms
    # butterfly tree: every lane sees the same sum -> rows sum to 1 within fp32 rounding
    assert np.abs(sm.astype(np.float64).sum(1) - 1.0).max() < 1e-5


def test_bf16_round_matches_torch_on_all_patterns():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    finite = np.isfinite(vals)
    np.testing.assert_array_equal(O.bf16_round(vals[finite]).view(np.uint32), bits[finite])
    rng = np.random.default_rng(1)
    # random fp32 bit patterns, including exact halfway cases
    raw = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    raw[:100000] = (raw[:100000] & 0xFFFF0000) | 0x8000
    f = raw.view(np.float32)
    f = f[np.isfinite(f)]
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(f).view(np.uint32), ref.view(np.uint32))


def test_combine_add_kat_sample():
    """bf16 + bf16 with fp32 opmath and one rounding (c2f_moe_combine_gate.py:54-84)."""

    rng = np.random.default_rng(2)
    a_bits = rng.integers(0, 1 << 16, size=4_000_000, dtype=np.uint32)
    b_bits = rng.integers(0, 1 << 16, size=4_000_000, dtype=np.uint32)
    a = O.bf16_bits_to_f32(a_bits.astype(np.uint16))
    b = O.bf16_bits_to_f32(b_bits.astype(np.uint16))
    ok = np.isfinite(a) & np.isfinite(b)
    a, b = a[ok], b[ok]
    ours = O.bf16_round((a + b).astype(np.float32))
    ta = torch.from_numpy(a.copy()).to(torch.bfloat16)
    tb = torch.from_numpy(b.copy()).to(torch.bfloat16)
    theirs = torch.add(ta, tb).float().numpy()
    fin = np.isfinite(theirs)
    np.testing.assert_array_equal(ours[fin].view(np.uint32), theirs[fin].view(np.uint32))


def test_fp8_e4m3_round_matches_torch():
    x = np.concatenate([
        np.linspace(-448.0, 448.0, 2_000_001, dtype=np.float32),
        (np.random.default_rng(3).standard_normal(1_000_000) * 20).clip(-448, 448).astype(np.float32),
        np.linspace(-0.05, 0.05, 100001, dtype=np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(O.fp8_e4m3_round(x), ref)


def test_fp8_codes_roundtrip():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    vals = O.fp8_e4m3_decode(codes)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(vals, ref)
    back = O.fp8_e4m3_encode(vals)
    # +0 / -0 both decode to zero; every other code round-trips
    nz = vals != 0
    np.testing.assert_array_equal(back[nz], codes[nz])
    # every int4 value is exact in e4m3
    q = np.arange(-8, 8, dtype=np.float32)
    np.testing.assert_array_equal(O.fp8_e4m3_round(q), q)


@pytest.mark.parametrize("amax", [1e-20, 1.0, 300.0])
def test_act_quant_per_token(amax):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((16, 512)) * amax).astype(np.float32)
    q, s = O.act_quant_per_token_fp8(x)
    assert np.abs(q).max() <= 448.0
    ref_s = np.maximum(np.abs(x).max(1, keepdims=True), np.float32(1e-12)) / np.float32(448.0)
    np.testing.assert_array_equal(s, ref_s.astype(np.float32))
    # closed form: q = e4m3(x / s), and the row max maps to +-448 exactly
    if amax >= 1.0:
        np.testing.assert_array_equal(np.abs(q).max(1), np.full(16, 448.0, dtype=np.float32))
        rel = np.abs(q * s - x).max() / np.abs(x).max()
        assert rel <= 2.0 ** -4
    else:
        # amax below the 1e-12 floor: x / s < 2^-10 rounds to zero in e4m3
        assert (q == 0).all()


def _bits(values):
    return O.bf16_to_bits(np.asarray(values, dtype=np.float32))


def test_running_sum_amplification_known_answers():
    """max_g (s_0 + ... + s_g) / s_g per row, by hand: equal scales -> the
    group count; an ascending row -> at most 2; a 2^100 group followed by a
    2^-100 group -> 2^200 (and the fp32 ratio of the two overflows)."""

    rows = np.stack([
        _bits([0.01] * 8),
        _bits([2.0 ** g for g in range(8)]),
        _bits([2.0 ** 100, 2.0 ** -100] + [1.0] * 6),
        _bits([1.0, 2.0 ** -70] + [1.0] * 6),
        _bits([1.0, 2.0 ** -60] + [1.0] * 6),
    ])
    amp = O.running_sum_amplification(rows)
    assert amp[0] == pytest.approx(8.0, rel=1e-2)          # bf16(0.01) repeated: exactly the group count
    assert 1.0 <= amp[1] <= 2.0
    assert amp[2] == pytest.approx(2.0 ** 200, rel=1e-6)
    assert amp[3] == pytest.approx(2.0 ** 70, rel=1e-6)
    assert amp[4] == pytest.approx(2.0 ** 60, rel=1e-6)
    flags = O.needs_exact_scaling(rows[:, None, :])          # five one-row matrices
    assert flags.tolist() == [False, False, True, True, False]
    # the whole matrix is marked when any one row is
    assert O.needs_exact_scaling(rows[None]).tolist() == [True]
    assert np.float32(2.0 ** 100) / np.float32(2.0 ** -100) == np.inf


def test_running_sum_overflow_is_what_the_rule_predicts():
    """A restatement of the running-sum recurrence in fp32 (a <- a * r + P,
    r = s[g-1] / s[g], result a * s[last]) against exact per-group scaling:
    finite and equal where the rule allows it, non-finite on a marked row."""

    def running(scales, partials):
        a = np.float32(0.0)
        for g, pg in enumerate(partials):
            r = np.float32(0.0) if g == 0 else np.float32(scales[g - 1]) / np.float32(scales[g])
            a = np.float32(a * r + np.float32(pg))
        return np.float32(a * np.float32(scales[-1]))

    partials = np.full(8, 2.0 ** 20, dtype=np.float32)
    safe = np.float32([1.0, 2.0 ** -40] + [1.0] * 6)
    wild = np.float32([2.0 ** 100, 2.0 ** -100] + [1.0] * 6)
    with np.errstate(over="ignore", invalid="ignore"):
        assert running(safe, partials) == pytest.approx(float((safe.astype(np.float64) * 2.0 ** 20).sum()), rel=1e-6)
        assert not np.isfinite(running(wild, partials))
    assert O.needs_exact_scaling(_bits(safe)[None, None]).tolist() == [False]
    assert O.needs_exact_scaling(_bits(wild)[None, None]).tolist() == [True]
