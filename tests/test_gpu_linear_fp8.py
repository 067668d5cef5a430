"""W8A16 dense linear over the reference checkpoint's FP8 format (E4M3 codes,
one E8M0 scale per 128 x 128 block): bf16 output against the fp32 closed form
C = A . bf16(Q * 2^(e-127))^T (oracle ``w8a16_fp8_linear_f32``, restating
``weight_only_linear.py:560-598`` and ``moe_forward.py:158-176``) to max_rel
and rel_fro <= 1e-2 at the benchmark shapes (K=4096, N in {4096, 1024, 16384},
M in {1, 64, 8192}), every split-K width and ragged M, N (last row block
partial).  A one-hot activation reads single weights back, which pins the
conversion bit for bit: byte order inside each lane, the scale block of every
strip and window, and scales from 2^-100 to 2^40.

Every case runs the reference's own entry (``w8a16_gemm_into`` on the
checkpoint's ``float8_e4m3fn`` weight and ``float8_e8m0fnu`` scales as
stored) and the load-time tiled variant (``w8a16_prepared_gemm_into``); the
two must give the same output bits.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import ops, synthetic as S
from gaiban_lite_amd import weight_only_linear as L
from helpers import assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def np_pack_bytes(q: np.ndarray) -> np.ndarray:
    """The 1 KiB tile layout (16 rows x 64 K, lane = 16j + row) of any 1-byte format."""

    n, k = q.shape
    t = q.reshape(n // 16, 16, k // 64, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(t).reshape(-1).view(np.uint8)


def run(m, n, k, *, split=None, seed=3, rows=None):
    print(f"[w8a16 fp8] M={m} N={n} K={k} split={split}", flush=True)
    codes, scales = S.make_fp8_block_linear(n, k, seed=seed, device=DEV)
    a = torch.randn((m, k), device=DEV, generator=torch.Generator(DEV).manual_seed(seed + 100)).to(torch.bfloat16)
    prep = L.prepare_fp8_block_weight(codes, scales)
    out = L.w8a16_linear(a, prep, split_k=split)
    raw = L.w8a16_linear(a, codes.view(torch.float8_e4m3fn), scales.view(torch.float8_e8m0fnu), split_k=split)
    torch.cuda.synchronize()
    assert torch.equal(raw, out), "checkpoint-layout and tiled weights differ"
    rows = np.arange(m) if rows is None else rows
    ref = O.w8a16_fp8_linear_f32(to_np_f32(a)[rows], codes.cpu().numpy(), scales.cpu().numpy())
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"fp8 M={m} N={n} split={split}")
    print(f"    {err}", flush=True)
    return out


def test_pack_fp8_layout():
    codes, _ = S.make_fp8_block_linear(64, 256, seed=5, device=DEV)
    packed = ops.pack_fp8(codes.view(torch.float8_e4m3fn))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(packed.cpu().numpy(), np_pack_bytes(codes.cpu().numpy()))


@pytest.mark.parametrize("split", [1, 4])
def test_one_hot_reads_back_every_weight_exactly(split):
    """out[i, n] = bf16(W[n, k_i]) for a one-hot row i of A: every E4M3 code,
    every byte position of a lane, every (row block, K block) scale."""

    n, k = 272, 512  # 3 row blocks (the last has 16 rows), 4 K blocks
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes
    codes[:254, 5] = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    scales = rng.integers(27, 168, size=(3, 4), dtype=np.uint8)  # 2^-100 .. 2^40
    scales[0, 0], scales[2, 3] = 27, 167
    cols = np.concatenate([np.arange(0, k, 7), [5, 63, 64, 127, 128, 511]])
    m = len(cols)
    a = np.zeros((m, k), dtype=np.float32)
    a[np.arange(m), cols] = 1.0
    at = torch.from_numpy(a).to(DEV).to(torch.bfloat16)
    codes_d, scales_d = torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV)
    prep = L.prepare_fp8_block_weight(codes_d, scales_d)
    out = L.w8a16_linear(at, prep, split_k=split)
    raw = L.w8a16_linear(at, codes_d.view(torch.float8_e4m3fn), scales_d.view(torch.float8_e8m0fnu), split_k=split)
    torch.cuda.synchronize()
    assert torch.equal(raw, out)
    # + 0.0: a sum that starts at +0 turns the -0 of code 0x80 into +0
    want = O.bf16_round(O.dequant_fp8_block(codes, scales))[:, cols].T + np.float32(0.0)
    got = to_np_f32(out)
    np.testing.assert_array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("n", [4096, 1024, 16384])
@pytest.mark.parametrize("m", [1, 64])
def test_decode_shapes(m, n):
    run(m, n, 4096)


@pytest.mark.parametrize("n", [4096, 1024, 16384])
def test_prefill_shapes_row_subset(n):
    rows = np.sort(np.random.default_rng(n).choice(8192, 96, replace=False))
    run(8192, n, 4096, rows=rows)


@pytest.mark.parametrize("split", [1, 2, 4, 8])
def test_every_split_width(split):
    run(64, 1024, 4096, split=split)


@pytest.mark.parametrize("m", [2, 17, 65, 129])
@pytest.mark.parametrize("n,k", [(48, 256), (208, 384), (1040, 1024)])
def test_ragged_shapes(m, n, k):
    run(m, n, k)
    run(m, n, k, split=2)


def test_scale_byte_zero_is_two_to_minus_127():
    """E8M0 byte 0 decodes to 2^-127 (weight_only_linear.py:503-513): the
    products are tiny but finite, and a block at 2^-127 next to normal blocks
    leaves the normal part exact."""

    n, k = 128, 256
    codes = np.full((n, k), 0x7E, dtype=np.uint8)  # 448
    scales = np.array([[0, 127]], dtype=np.uint8)   # 2^-127 | 1.0
    a = np.zeros((2, k), dtype=np.float32)
    a[0, 3] = 1.0      # reads a weight of the 2^-127 block
    a[1, 200] = 1.0    # reads a weight of the unit block
    prep = L.prepare_fp8_block_weight(torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV))
    out = to_np_f32(L.w8a16_linear(torch.from_numpy(a).to(DEV).to(torch.bfloat16), prep))
    torch.cuda.synchronize()
    assert np.isfinite(out).all()
    np.testing.assert_array_equal(out[1], np.full(n, 448.0, dtype=np.float32))
    ref0 = 448.0 * 2.0 ** -127
    assert np.all(np.abs(out[0] - ref0) <= ref0 * 2.0 ** -6)


@pytest.mark.parametrize("split", [2, 4])
def test_prefill_tile_with_explicit_split(split):
    """The 256 x 128 prefill tile (weights three buffers deep) over a K split."""

    rows = np.sort(np.random.default_rng(split).choice(8192, 64, replace=False))
    run(8192, 4096, 4096, split=split, rows=rows)


def test_reference_call_sequence():
    """The reference module's own sequence (``weight_only_linear.py:182-221,
    406-513,794-823``): plan, metadata validation, non-alias preflight, the
    E8M0 preflight, then the hot call into caller-owned storage, repeated
    without allocation; bad calls raise before any launch."""

    m, n, k = 64, 1024, 4096
    codes, scales = S.make_fp8_block_linear(n, k, seed=9, device=DEV)
    weight, scale = codes.view(torch.float8_e4m3fn), scales.view(torch.float8_e8m0fnu)
    a = torch.randn((m, k), device=DEV, generator=torch.Generator(DEV).manual_seed(9)).to(torch.bfloat16)
    plan = L.make_gemm_plan(m, n, k)
    out = torch.empty(plan.output_shape, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(plan.workspace_shape, dtype=torch.float32, device=DEV)
    assert plan.weight_shape == (n, k) and plan.weight_scale_shape == (n // 128, k // 128)
    L.validate_fp8_weight_only_tensors(a, weight, scale, out, ws, plan=plan)
    L.validate_non_alias_tensors({"activation": a, "weight": weight, "weight_scale": scale, "out": out,
                                  "workspace": ws})
    L.validate_e8m0_scale_values("weight_scale", scale)
    L.w8a16_gemm_into(a, weight, scale, out, ws, plan=plan)
    first = out.clone()
    L.fp8_weight_only_linear_into(a, weight, scale, out, ws, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(out, first)
    ref = O.w8a16_fp8_linear_f32(to_np_f32(a), codes.cpu().numpy(), scales.cpu().numpy())
    assert_moe_close(to_np_f32(out), ref, what="reference sequence")
    with pytest.raises(TypeError):  # tiled bytes are not the checkpoint contract
        L.w8a16_gemm_into(a, codes, scale, out, ws, plan=plan)
    with pytest.raises(TypeError):
        L.w8a16_gemm_into(a, weight, scales, out, ws, plan=plan)
    with pytest.raises(ValueError):
        L.validate_non_alias_tensors({"out": out, "alias": out[:1]})
