"""CPU pins of the block-FP8 W8A8 oracle (``fp8_linear.py:354-424``).

``act_quant_block_fp8`` against an independent torch statement: the scale as
2^ceil(log2(max(amax, 1e-4) * fp32(1/448))) and torch's own float8_e4m3fn
cast.  ``block_fp8_gemm_f32`` against a float64 matmul of operands that were
dequantised first (the scales applied to A and W instead of to each block
product), which fails if a block index, a scale row or an operand is off."""

import numpy as np
import torch

import oracle as O


def torch_quant(x: np.ndarray):
    m, k = x.shape
    xt = torch.from_numpy(x).view(m, k // 128, 128)
    su = torch.clamp(xt.abs().amax(-1), min=1e-4) * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    e = torch.ceil(torch.log2(su.double()))
    s = torch.exp2(e).float()
    q = (xt / s[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).reshape(m, k)
    return q.numpy(), (e + 127).to(torch.uint8).numpy()


def test_act_quant_matches_torch_statement():
    rng = np.random.default_rng(0)
    mags = np.array([1.0, 1e-3, 100.0, 1e-8, 3e4, 1e30, 2.0**-126, 448.0])
    x = (rng.standard_normal((8, 512)) * mags[:, None]).astype(np.float32)
    x[1, :128] = 0.0                       # an all-zero block: amax floor 1e-4
    x[2, 128:256] = 448.0 * 2.0**-7        # exactly a power-of-two multiple of 448
    x[3, 256] = -np.float32(3.0e38)        # the largest magnitudes
    q, e = O.act_quant_block_fp8(x)
    tq, te = torch_quant(x)
    np.testing.assert_array_equal(e, te)
    np.testing.assert_array_equal(q, tq)
    assert e.min() >= 1 and e.max() <= 254


def test_act_quant_bf16_inputs_and_round_trip_bound():
    rng = np.random.default_rng(1)
    x = O.bf16_round(rng.standard_normal((16, 1024)).astype(np.float32) * 3.0)
    q, e = O.act_quant_block_fp8(x)
    tq, te = torch_quant(x)
    np.testing.assert_array_equal(q, tq)
    np.testing.assert_array_equal(e, te)
    # dequantised values stay within half an e4m3 ulp (2^-4 relative) of x
    deq = O.fp8_e4m3_decode(q).reshape(16, 8, 128) * O.decode_e8m0(e)[..., None]
    err = np.abs(deq.reshape(16, 1024) - x)
    assert np.all(err <= np.abs(x) * 2.0**-4 + O.decode_e8m0(e).repeat(128, axis=1) * 2.0**-10)


def test_block_gemm_against_dequantised_matmul():
    rng = np.random.default_rng(2)
    m, n, k = 7, 272, 512                  # 3 weight row blocks, the last partial
    a_codes, a_scale = O.act_quant_block_fp8(rng.standard_normal((m, k)).astype(np.float32))
    w_codes = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    w_codes[(w_codes & 0x7F) == 0x7F] = 0x38
    w_scale = rng.integers(100, 140, size=(3, k // 128), dtype=np.uint8)
    got = O.block_fp8_gemm_f32(a_codes, a_scale, w_codes, w_scale)
    a = O.fp8_e4m3_decode(a_codes).astype(np.float64) * np.repeat(O.decode_e8m0(a_scale), 128, axis=1)
    w = O.dequant_fp8_block(w_codes, w_scale).astype(np.float64)
    want = a @ w.T
    np.testing.assert_allclose(got, want.astype(np.float32), rtol=1e-6, atol=1e-30)
    # a planted mistake fails: the scale of the wrong weight row block
    bad = w_scale.copy()
    bad[[0, 1]] = bad[[1, 0]]
    assert not np.allclose(O.block_fp8_gemm_f32(a_codes, a_scale, w_codes, bad), want, rtol=1e-3)
