"""W8A16 dense linear: bf16 output against the fp32 closed form
C = A . (Q * s)^T (oracle ``w8a16_linear_f32``) on seeded inputs, to max_rel
and rel_fro <= 1e-2, at the benchmark shapes (K=4096, N in {4096, 1024,
16384}, M in {1, 64, 8192}), every split-K width, ragged M and N, and the
tiled packer against an independent numpy statement of its layout.

Every case runs twice: on the int8 weight as stored (row-major [N, K],
``w8a16_int8_gemm_into``) and on the load-time tiles (``prepare_int8_weight``,
``w8a16_prepared_gemm_into``); the two must give the same output bits.

Rows of C depend only on the same row of A, so M=8192 is checked on a seeded
subset of rows (the kernel still computes all of them).
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import ops, synthetic as S
from gaiban_lite_amd import weight_only_linear as L
from helpers import assert_moe_close, bf16_bits, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def np_pack_int8(q: np.ndarray) -> np.ndarray:
    n, k = q.shape
    t = q.reshape(n // 16, 16, k // 64, 4, 16)          # strip, row, window, j, byte
    t = t.transpose(0, 2, 3, 1, 4)                       # strip, window, j, row, byte -> lane = 16j + row
    return np.ascontiguousarray(t).reshape(-1).view(np.uint8)


def run(m, n, k, *, split=None, seed=3, rows=None):
    print(f"[w8a16] M={m} N={n} K={k} split={split}", flush=True)
    q, s = S.make_int8_linear(n, k, seed=seed, device=DEV)
    a = torch.randn((m, k), device=DEV, generator=torch.Generator(DEV).manual_seed(seed + 100)).to(torch.bfloat16)
    prep = L.prepare_int8_weight(q, s)
    out = L.w8a16_linear(a, prep, split_k=split)
    raw = L.w8a16_linear(a, q, s, split_k=split)
    torch.cuda.synchronize()
    assert torch.equal(raw, out), "row-major and tiled weights differ"
    rows = np.arange(m) if rows is None else rows
    ref = O.w8a16_linear_f32(to_np_f32(a)[rows], q.cpu().numpy(), bf16_bits(s))
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"M={m} N={n} split={split}")
    print(f"    {err}", flush=True)
    return out


def test_pack_int8_layout():
    q, _ = S.make_int8_linear(64, 256, seed=5, device=DEV)
    packed = ops.pack_int8(q)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(packed.cpu().numpy(), np_pack_int8(q.cpu().numpy()))


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
    out = run(64, 1024, 4096, split=split)
    base = run(64, 1024, 4096, split=1) if split != 1 else out
    # a different split only changes the fp32 summation order
    d = (out.float() - base.float()).abs().max().item()
    assert d <= 2e-2 * base.float().abs().max().item()


@pytest.mark.parametrize("m", [2, 3, 17, 33, 65, 100, 129])
@pytest.mark.parametrize("n,k", [(48, 256), (208, 384)])
def test_ragged_shapes(m, n, k):
    run(m, n, k)
    run(m, n, k, split=2)


def test_zero_rows_and_contract_errors():
    q, s = S.make_int8_linear(64, 256, device=DEV)
    prep = L.prepare_int8_weight(q, s)
    a = torch.empty((0, 256), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((0, 64), dtype=torch.bfloat16, device=DEV)
    ops.w8a16_linear_into(a, prep.packed, prep.scale, out, None, n=64, split_k=1)
    ops.w8a16_linear_into(a, q, s, out, None, n=64, split_k=1)
    plan = L.make_gemm_plan(4, 64, 256, split_k=2)
    a = torch.zeros((4, 256), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((4, 64), dtype=torch.bfloat16, device=DEV)
    ws = L.allocate_workspace(plan, DEV)
    with pytest.raises(ValueError):  # workspace shape
        L.w8a16_int8_gemm_into(a, q, s, out, torch.empty((1, 4, 64), dtype=torch.float32, device=DEV), plan=plan)
    with pytest.raises(ValueError):
        L.w8a16_prepared_gemm_into(a, prep, out, torch.empty((1, 4, 64), dtype=torch.float32, device=DEV),
                                   plan=plan)
    with pytest.raises(TypeError):  # activation dtype
        L.w8a16_int8_gemm_into(a.float(), q, s, out, ws, plan=plan)
    with pytest.raises(TypeError):  # weight dtype
        L.w8a16_int8_gemm_into(a, q.view(torch.uint8), s, out, ws, plan=plan)
    with pytest.raises(ValueError):  # weight shape
        L.w8a16_int8_gemm_into(a, q[:32], s, out, ws, plan=plan)
    with pytest.raises(TypeError):  # an int8 weight is not the checkpoint FP8 contract
        L.w8a16_gemm_into(a, q, s, out, ws, plan=plan)
    with pytest.raises(ValueError):
        L.make_gemm_plan(4, 64, 200)
    with pytest.raises(ValueError):
        L.make_gemm_plan(4, 64, 256, split_k=4)  # 2 K-blocks


def test_prefill_tile_with_explicit_split():
    """The 256 x 128 prefill tile (weights three buffers deep) over a K split."""

    rows = np.sort(np.random.default_rng(7).choice(8192, 64, replace=False))
    run(8192, 4096, 4096, split=2, rows=rows)


@pytest.mark.parametrize("m,n,k,split", [(1, 4096, 4096, 8), (2, 1024, 4096, 2), (3, 16384, 4096, 4),
                                         (4, 4096, 1024, 8), (5, 1024, 4096, 4), (16, 4096, 4096, 2),
                                         (24, 1024, 4096, 8), (33, 4096, 4096, 4), (64, 1024, 4096, 8),
                                         (64, 16384, 4096, 4), (3, 208, 640, 4), (40, 208, 640, 4),
                                         (48, 4096, 4096, 8), (20, 208, 2048, 8)])
@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_in_workgroup_split_matches_two_launch_reduction(m, n, k, split, fmt):
    """Up to 64 tokens a K split runs inside one workgroup (each wavefront
    one split's partial, summed through LDS in split order); above 64 the
    partials go through the workspace and a reduce launch (17..64 tokens with
    4 or 8 windows per split: weights straight to registers, the split's
    token rows in LDS).  A row of C
    depends only on its row of A, and the split boundaries are the same, so
    the first m rows of a 128-token call with the same split must carry the
    same bits -- which pins the in-workgroup order of the additions.  Up to
    4 tokens with splits covering K exactly the activation rows go through
    LDS (M=1..4 here); ragged N and a last split shorter than the others
    included (K=640: 10 windows over 4 splits of 3)."""

    print(f"[w8a16 {fmt}] in-workgroup split M={m} N={n} K={k} split={split}", flush=True)
    gen = torch.Generator(DEV).manual_seed(m * 7 + split)
    a = torch.randn((128, k), device=DEV, generator=gen).to(torch.bfloat16)
    if fmt == "fp8":
        codes, scales = S.make_fp8_block_linear(n, k, seed=31, device=DEV)
        w, w_s = codes.view(torch.float8_e4m3fn), scales.view(torch.float8_e8m0fnu)
        prep = L.prepare_fp8_block_weight(codes, scales)
    else:
        w, w_s = S.make_int8_linear(n, k, seed=31, device=DEV)
        prep = L.prepare_int8_weight(w, w_s)
    small = L.w8a16_linear(a[:m].contiguous(), w, w_s, split_k=split)
    small_tiled = L.w8a16_linear(a[:m].contiguous(), prep, split_k=split)
    big = L.w8a16_linear(a, w, w_s, split_k=split)
    torch.cuda.synchronize()
    assert torch.equal(small.view(torch.int16), small_tiled.view(torch.int16))
    assert torch.equal(small.view(torch.int16), big[:m].view(torch.int16))
