"""Pins the oracle's weight formats, expert FFN, W8A16 and split-K policy with
known answers, scalar loops on tiny shapes and algebraic properties."""

import numpy as np
import pytest

import oracle as O


def test_int4_pack_known_answer():
    q = np.array([[0, 1, -1, 7, -8, 3, 2, -2]], dtype=np.int8)
    p = O.pack_int4_rows(q)
    # byte b: low nibble = k=2b, high nibble = k=2b+1, two's complement
    np.testing.assert_array_equal(p, np.array([[0x10, 0x7F, 0x38, 0xE2]], dtype=np.uint8))
    np.testing.assert_array_equal(O.unpack_int4_rows(p), q)


def test_int4_roundtrip_and_group_indexing():
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, size=(32, 512)).astype(np.int8)
    p = O.pack_int4_rows(q)
    np.testing.assert_array_equal(O.unpack_int4_rows(p), q)
    s = O.bf16_round(rng.uniform(0.005, 0.02, size=(32, 4)).astype(np.float32))
    w = O.dequant_int4_g128(p, O.bf16_to_bits(s))
    for n in (0, 7, 31):
        for k in (0, 127, 128, 300, 511):
            assert w[n, k] == np.float32(q[n, k]) * s[n, k // 128]


def test_fp4_table_and_e8m0_known_answers():
    # moe_forward.py:23-40 (identical tables in convert.py:11-14, common.py:42-44)
    assert O.FP4_VALUES == (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                            0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)
    # weight_only_linear.py:503-513: byte 0 -> 2^-127, b -> 2^(b-127)
    codes = np.array([0, 1, 127, 128, 254], dtype=np.uint8)
    np.testing.assert_array_equal(O.decode_e8m0(codes),
                                  np.array([2.0 ** -127, 2.0 ** -126, 1.0, 2.0, 2.0 ** 127], dtype=np.float32))
    with pytest.raises(ValueError):
        O.decode_e8m0(np.array([255], dtype=np.uint8))
    packed = np.array([[0x21, 0xF9] + [0] * 14], dtype=np.uint8)  # 32 values, one scale
    w = O.dequant_mxfp4(packed, np.array([[128]], dtype=np.uint8))
    np.testing.assert_array_equal(w[0, :4], np.array([1.0, 2.0, -1.0, -12.0], dtype=np.float32))


def test_mxfp4_dequant_is_exact_in_bf16():
    """c2f-dense-gate.json dequant_bf16_exact: E2M1 x E8M0 needs <= 3 significand bits."""

    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, size=(64, 128), dtype=np.uint8)
    sc = rng.integers(100, 150, size=(64, 8), dtype=np.uint8)
    w = O.dequant_mxfp4(packed, sc)
    np.testing.assert_array_equal(O.bf16_round(w), w)


def _tiny_source(rng, e, h, i):
    w13 = rng.integers(0, 256, size=(e, 2 * i, h // 2), dtype=np.uint8)
    s13 = O.bf16_to_bits(rng.uniform(0.005, 0.02, size=(e, 2 * i, h // 128)).astype(np.float32))
    w2 = rng.integers(0, 256, size=(e, h, i // 2), dtype=np.uint8)
    s2 = O.bf16_to_bits(rng.uniform(0.005, 0.02, size=(e, h, i // 128)).astype(np.float32))
    return O.ExpertSource(w13, s13, w2, s2)


@pytest.mark.parametrize("clamp", [0.0, 0.3])
def test_moe_fp32_matches_scalar_loops(clamp):
    rng = np.random.default_rng(2)
    e, h, i, t, k = 3, 128, 128, 4, 2
    src = _tiny_source(rng, e + 1, h, i)
    x = O.bf16_round(rng.standard_normal((t, h)).astype(np.float32))
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1]])
    w = rng.uniform(0.1, 1.0, size=(t, k)).astype(np.float32)
    got = O.moe_fp32(x, ids, w, src, shared_index=e, clamp_limit=clamp)
    ref = np.zeros((t, h), dtype=np.float64)

    def ffn(tok, ex, weight):
        w13 = src.w13(ex).astype(np.float64)
        w2 = src.w2(ex).astype(np.float64)
        act = np.zeros(i)
        for n in range(i):
            g = sum(x[tok, c] * w13[n, c] for c in range(h))
            u = sum(x[tok, c] * w13[i + n, c] for c in range(h))
            if clamp > 0:
                g = min(g, clamp)
                u = min(max(u, -clamp), clamp)
            act[n] = g / (1 + np.exp(-g)) * u * weight
        return np.array([sum(act[n] * w2[m, n] for n in range(i)) for m in range(h)])

    for tok in range(t):
        for j in range(k):
            ref[tok] += ffn(tok, ids[tok, j], w[tok, j])
        ref[tok] += ffn(tok, e, 1.0)
    np.testing.assert_allclose(got, ref, rtol=2e-4, atol=2e-4 * np.abs(ref).max())


def test_moe_fp32_linear_in_route_weights_and_row_subset():
    rng = np.random.default_rng(3)
    src = _tiny_source(rng, 4, 256, 128)
    x = rng.standard_normal((10, 256)).astype(np.float32)
    ids = np.argsort(rng.random((10, 4)), axis=1)[:, :2]
    w = rng.uniform(0.1, 1.0, size=(10, 2)).astype(np.float32)
    y1 = O.moe_fp32(x, ids, w, src)
    y2 = O.moe_fp32(x, ids, 2 * w, src)
    np.testing.assert_allclose(y2, 2 * y1, rtol=1e-5, atol=1e-5 * np.abs(y1).max())
    sub = O.moe_fp32(x, ids, w, src, rows=[3, 7])
    np.testing.assert_allclose(sub, y1[[3, 7]], rtol=1e-6, atol=1e-6)


def test_bf16_mirror_close_to_fp32_oracle():
    rng = np.random.default_rng(4)
    src = _tiny_source(rng, 5, 512, 256)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    ids = np.argsort(rng.random((16, 4)), axis=1)[:, :2]
    w = rng.uniform(0.2, 0.8, size=(16, 2)).astype(np.float32)
    a = O.moe_bf16_mirror(x, ids, w, src, shared_index=4)
    b = O.moe_fp32(O.bf16_round(x), ids, w, src, shared_index=4)
    assert O.rel_fro(a, b) < 1e-2
    np.testing.assert_array_equal(O.bf16_round(a), a)
    c = O.moe_bf16_mirror(x, ids, w, src, shared_index=4, workers=4)
    np.testing.assert_array_equal(a, c)


def test_w8a16_oracle_and_split_k_policy():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((3, 256)).astype(np.float32)
    q = rng.integers(-127, 128, size=(5, 256)).astype(np.int8)
    s = O.bf16_round(rng.uniform(0.005, 0.02, size=5).astype(np.float32))
    got = O.w8a16_linear_f32(a, q, O.bf16_to_bits(s))
    ref = np.array([[sum(float(a[m, c]) * float(q[n, c]) * float(s[n]) for c in range(256))
                     for n in range(5)] for m in range(3)])
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # weight_only_linear.py:168-179 with block 32 x 64 (tiles = ceil(m/32)*ceil(n/64), kb = k/128)
    assert O.automatic_split_k(1, 1024, 4096) == 4      # 16 tiles < 32, 32 K blocks
    assert O.automatic_split_k(1, 4096, 4096) == 2      # 64 tiles < 96, >= 16 K blocks
    assert O.automatic_split_k(64, 1024, 4096) == 2     # 32 tiles
    assert O.automatic_split_k(1, 1024, 2048) == 2      # 16 K blocks only
    assert O.automatic_split_k(1, 1024, 1024) == 1      # 8 K blocks
    assert O.automatic_split_k(64, 16384, 4096) == 1
    assert O.automatic_split_k(8192, 4096, 4096) == 1


def test_moe_w4a8_oracle_against_torch_fp8_pipeline():
    """W4A8 oracle vs an independent float64 pipeline whose fp8 rounding is
    torch's float8_e4m3fn cast: per-token quant of x, fp32->bf16 SwiGLU,
    per-row quant of h, route weight on the w2 output, shared expert weight 1."""

    import torch

    rng = np.random.default_rng(9)
    e, h, i, t, k = 3, 128, 128, 5, 2
    src = _tiny_source(rng, e + 1, h, i)
    x = O.bf16_round((rng.standard_normal((t, h)) * 3).astype(np.float32))
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1], [2, 0]])
    w = rng.uniform(0.1, 1.0, size=(t, k)).astype(np.float32)
    got = O.moe_w4a8_f32(x, ids, w, src, shared_index=e, clamp_limit=0.4)

    def quant(v):
        v = torch.from_numpy(np.asarray(v, dtype=np.float32))
        s = v.abs().amax(-1, keepdim=True).clamp_min(1e-12) / 448.0
        q = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float64)
        return (q * s.double()).numpy()

    xd = quant(x)
    ref = np.zeros((t, h))
    for tok in range(t):
        pairs = [(ids[tok, j], float(w[tok, j])) for j in range(k)] + [(e, 1.0)]
        for ex, weight in pairs:
            w13 = src.w13(ex).astype(np.float64)
            g = np.minimum(xd[tok] @ w13[:i].T, 0.4)
            u = np.clip(xd[tok] @ w13[i:].T, -0.4, 0.4)
            act = torch.from_numpy((g / (1 + np.exp(-g)) * u).astype(np.float32)).to(torch.bfloat16).float().numpy()
            ref[tok] += (quant(act[None])[0] @ src.w2(ex).astype(np.float64).T) * weight
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    # the quantisation is not the identity: the W4A8 result differs from the W4A16 one
    assert O.rel_fro(got, O.moe_fp32(x, ids, w, src, shared_index=e, clamp_limit=0.4)) > 1e-3


def test_moe_w4a8_mxfp4_oracle_against_torch_fp8_pipeline():
    """MXFP4 W4A8 oracle vs an independent float64 pipeline: torch's
    float8_e4m3fn cast for x and h, the MXFP4 weights dequantised by the
    torch restatement of the reference's table lookup (``torch_path.
    dequant_mxfp4``), E8M0 scales spread over 2^-30 .. 2^10 per 32-K group."""

    import torch

    from oracle import torch_path as TP

    rng = np.random.default_rng(19)
    e, h, i, t, k = 3, 256, 128, 5, 2
    w13 = rng.integers(0, 256, size=(e + 1, 2 * i, h // 2), dtype=np.uint8)
    s13 = rng.integers(97, 138, size=(e + 1, 2 * i, h // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, size=(e + 1, h, i // 2), dtype=np.uint8)
    s2 = rng.integers(97, 138, size=(e + 1, h, i // 32), dtype=np.uint8)
    src = O.MXFP4ExpertSource(w13, s13, w2, s2)
    x = O.bf16_round((rng.standard_normal((t, h)) * 3).astype(np.float32))
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1], [2, 0]])
    w = rng.uniform(0.1, 1.0, size=(t, k)).astype(np.float32)
    got = O.moe_w4a8_mxfp4_f32(x, ids, w, src, shared_index=e, clamp_limit=0.0)

    def quant(v):
        v = torch.from_numpy(np.asarray(v, dtype=np.float32))
        s = v.abs().amax(-1, keepdim=True).clamp_min(1e-12) / 448.0
        q = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float64)
        return (q * s.double()).numpy()

    def deq(codes, scales):
        return TP.dequant_mxfp4(torch.from_numpy(codes), torch.from_numpy(scales)).double().numpy()

    xd = quant(x)
    ref = np.zeros((t, h))
    for tok in range(t):
        pairs = [(ids[tok, j], float(w[tok, j])) for j in range(k)] + [(e, 1.0)]
        for ex, weight in pairs:
            m13 = deq(w13[ex], s13[ex])
            g = xd[tok] @ m13[:i].T
            u = xd[tok] @ m13[i:].T
            act = torch.from_numpy((g / (1 + np.exp(-g)) * u).astype(np.float32)).to(torch.bfloat16).float().numpy()
            ref[tok] += (quant(act[None])[0] @ deq(w2[ex], s2[ex]).T) * weight
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    assert O.rel_fro(got, O.moe_fp32(x, ids, w, src, shared_index=e)) > 1e-3
    with pytest.raises(TypeError):
        O.moe_w4a8_mxfp4_f32(x, ids, w, _tiny_source(rng, e + 1, 128, 128))


def test_e8m0_decode_matches_torch_float8_e8m0fnu():
    """The reference decodes scales with scale.view(torch.float8_e8m0fnu).float()
    (moe_forward.py:115-123); the oracle's decode equals it for every byte but
    the reserved 255 (NaN there, rejected here)."""

    import torch

    codes = np.arange(255, dtype=np.uint8)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e8m0fnu).float().numpy()
    np.testing.assert_array_equal(O.decode_e8m0(codes), ref)
    assert np.isnan(torch.tensor([255], dtype=torch.uint8).view(torch.float8_e8m0fnu).float().item())


def test_mxfp4_source_is_dequant_then_matmul():
    """MXFP4ExpertSource dequantises with dequant_mxfp4 (w13 rows = gate, up)."""

    rng = np.random.default_rng(5)
    e, h, i = 2, 256, 128
    w13 = rng.integers(0, 256, size=(e, 2 * i, h // 2), dtype=np.uint8)
    s13 = rng.integers(118, 124, size=(e, 2 * i, h // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, size=(e, h, i // 2), dtype=np.uint8)
    s2 = rng.integers(118, 124, size=(e, h, i // 32), dtype=np.uint8)
    src = O.MXFP4ExpertSource(w13, s13, w2, s2)
    table = np.asarray(O.FP4_VALUES, dtype=np.float32)
    for ex in range(e):
        w = src.w13(ex)
        for n, k in ((0, 0), (5, 33), (2 * i - 1, h - 1)):
            code = (w13[ex, n, k // 2] >> (4 * (k % 2))) & 0xF
            assert w[n, k] == table[code] * np.float32(2.0 ** (int(s13[ex, n, k // 32]) - 127))
        assert src.w2(ex).shape == (h, i)


def test_fp8_block_dequant_matches_torch_fp8_dtypes():
    """dequant_fp8_block (moe_forward.py:158-176) = torch's float8_e4m3fn decode
    times torch's float8_e8m0fnu decode of the block's scale, including a
    ragged last row block, scale byte 0 (2^-127) and every finite E4M3 code."""

    import torch

    rng = np.random.default_rng(11)
    n, k = 300, 384  # 3 row blocks (the last holds 44 rows), 3 K blocks
    codes = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    codes[0, :254] = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    scales = rng.integers(100, 140, size=(3, 3), dtype=np.uint8)
    scales[1, 2] = 0
    scales[2, 0] = 254
    got = O.dequant_fp8_block(codes, scales)
    w = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float()
    s = torch.from_numpy(scales.copy()).view(torch.float8_e8m0fnu).float()
    ref = (w * s.repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]).numpy()
    np.testing.assert_array_equal(got, ref)
    with pytest.raises(ValueError):
        O.dequant_fp8_block(codes, scales[:2])


def test_w8a16_fp8_linear_oracle_against_scalar_loop():
    """A . bf16(Q * 2^(e-127))^T (weight_only_linear.py:583-590) on a tiny shape."""

    rng = np.random.default_rng(12)
    a = O.bf16_round(rng.standard_normal((3, 256)).astype(np.float32))
    codes = rng.integers(0, 0x7E, size=(5, 256), dtype=np.uint8)  # positive finite E4M3
    codes[::2] |= 0x80                                           # and some negative
    scales = np.array([[120, 131]], dtype=np.uint8)
    got = O.w8a16_fp8_linear_f32(a, codes, scales)
    dec = O.fp8_e4m3_decode(codes)
    ref = np.zeros((3, 5))
    for m in range(3):
        for n_ in range(5):
            for c in range(256):
                wv = float(O.bf16_round(np.array([dec[n_, c] * 2.0 ** (int(scales[0, c // 128]) - 127)],
                                                 dtype=np.float32))[0])
                ref[m, n_] += float(a[m, c]) * wv
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_shared_fp8_oracle_matches_reference_op_order_in_torch():
    """shared_fp8_bf16 equals the reference's torch sequence
    (moe_runtime.py:238-263: dequant_fp8_block -> bf16, F.linear in bf16,
    .float().clamp, F.silu, .to(bf16), F.linear) bit for bit.  Operands are
    small dyadic values, so every fp32 sum is exact and the accumulation order
    cannot matter; gate and up exceed the clamp for some entries."""

    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(21)
    t, h, i, lim = 5, 256, 128, 3.0
    enc = O.fp8_e4m3_encode
    vals = np.array([-8, -4, -3, -2, -1, -0.5, 0, 0.5, 1, 2, 3, 4, 8], dtype=np.float32)
    w1 = enc(rng.choice(vals, size=(i, h)).astype(np.float32))
    w3 = enc(rng.choice(vals, size=(i, h)).astype(np.float32))
    w2 = enc(rng.choice(vals, size=(h, i)).astype(np.float32))
    s1 = np.full((1, 2), 123, dtype=np.uint8)   # 2^-4
    s3 = np.array([[124, 122]], dtype=np.uint8)
    s2 = np.full((2, 1), 121, dtype=np.uint8)
    x = (rng.integers(-4, 5, size=(t, h)) * 0.25).astype(np.float32)
    got = O.shared_fp8_bf16(x, w1, s1, w3, s3, w2, s2, lim)

    def dq(c, s):
        wv = torch.from_numpy(c.copy()).view(torch.float8_e4m3fn).float()
        sv = torch.from_numpy(s.copy()).view(torch.float8_e8m0fnu).float()
        return (wv * sv.repeat_interleave(128, 0).repeat_interleave(128, 1)).to(torch.bfloat16)

    xb = torch.from_numpy(x).to(torch.bfloat16)
    gate = F.linear(xb, dq(w1, s1)).float().clamp(max=lim)
    up = F.linear(xb, dq(w3, s3)).float().clamp(min=-lim, max=lim)
    assert float(gate.max()) == lim and float(up.abs().max()) == lim  # the clamps bite
    act = (F.silu(gate) * up).to(torch.bfloat16)
    ref = F.linear(act, dq(w2, s2)).float().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=0)


@pytest.mark.parametrize("limit", [0.0, 10.0])
def test_swiglu_against_torch_expert_activation(limit):
    """``swiglu_f32`` vs torch's own ops in ``Expert.forward``'s order
    (``model.py:598-603``): up clamped to [-limit, limit], gate clamped above
    only, then ``F.silu(gate) * up`` in fp32.  Inputs reach +-40, so a
    missing clamp, a gate clamped below as well, or an up clamped on one
    side only moves outputs far beyond the tolerance (checked below)."""

    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(23)
    g = (rng.standard_normal((64, 96)) * 15).astype(np.float32)
    u = (rng.standard_normal((64, 96)) * 15).astype(np.float32)
    g[0, :4] = [-40.0, 40.0, 0.0, -0.0]
    u[0, :4] = [-40.0, 40.0, 1.0, 1.0]

    def torch_ref(gg, uu, lim, gate_min=False, up_max_only=False):
        gt, ut = torch.from_numpy(gg), torch.from_numpy(uu)
        if lim > 0:
            ut = torch.clamp(ut, max=lim) if up_max_only else torch.clamp(ut, min=-lim, max=lim)
            gt = torch.clamp(gt, min=-lim, max=lim) if gate_min else torch.clamp(gt, max=lim)
        return (F.silu(gt) * ut).numpy()

    got = O.swiglu_f32(g, u, limit)
    ref = torch_ref(g, u, limit)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-30)
    if limit > 0:
        for wrong in (torch_ref(g, u, 0.0), torch_ref(g, u, limit, gate_min=True),
                      torch_ref(g, u, limit, up_max_only=True)):
            assert not np.allclose(got, wrong, rtol=1e-3, atol=1e-6)
