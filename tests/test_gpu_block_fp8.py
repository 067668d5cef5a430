"""Block-FP8 W8A8 dense linear (``runtime/dsv4_direct/fp8_linear.py``): the
activation quantiser bit for bit against the oracle ``act_quant_block_fp8``
(itself pinned to torch's float8 cast on the CPU), and the GEMM against the
exact-product closed form ``block_fp8_gemm_f32`` to max_rel and rel_fro <=
1e-2 at the benchmark shapes (K=4096, N in {1024, 4096, 16384}, M in {1, 64,
8192}), every split, ragged M / N / K.  A one-hot activation with a distinct
E8M0 scale per (token, K block) reads single weights back exactly, which pins
the byte order of both operands, the weight row block, and which lane's scale
the MFMA applies to which token and K block."""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import fp8_linear as F
from gaiban_lite_amd import ops, synthetic as S
from gaiban_lite_amd import weight_only_linear as L
from helpers import assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def quant(x: torch.Tensor):
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    s = torch.empty((m, k // 128), dtype=torch.uint8, device=DEV)
    ops.act_quant_block_fp8_into(x, q, s)
    return q, s


def gemm(q, s, prep, split=None, raw=None):
    """The GEMM over the prepared tiles, or with ``raw`` (the E4M3 [n, k]
    bytes as stored) over the checkpoint layout."""
    m, k = q.shape
    split = ops.block_fp8_split_k(m, prep.n, k) if split is None else split
    out = torch.empty((m, prep.n), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(ops.block_fp8_workspace_bytes(m, prep.n, split) // 4, 1), dtype=torch.float32, device=DEV)
    ops.block_fp8_gemm_into(q, s, prep.packed if raw is None else raw, prep.scale, out, ws, n=prep.n, split_k=split)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k", [(1, 128), (7, 512), (64, 4096), (300, 1024)])
def test_act_quant_bit_exact(dtype, m, k):
    print(f"[block fp8] quant {dtype} m={m} k={k}", flush=True)
    g = torch.Generator(DEV).manual_seed(m + k)
    mags = torch.logspace(-9, 4, m, device=DEV) if m > 1 else torch.ones(1, device=DEV)
    x = (torch.randn((m, k), device=DEV, generator=g) * mags[:, None]).to(dtype)
    if m >= 7:
        x[2, :128] = 0      # all-zero block: the 1e-4 amax floor
        x[3, 5] = 60000.0 if dtype == torch.float16 else 1e30
    q, s = quant(x)
    torch.cuda.synchronize()
    want_q, want_s = O.act_quant_block_fp8(x.float().cpu().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)


def test_act_quant_prefill_shape():
    print("[block fp8] quant 8192 x 4096", flush=True)
    x = S.make_hidden(8192, 4096, seed=3, device=DEV)
    q, s = quant(x)
    torch.cuda.synchronize()
    want_q, want_s = O.act_quant_block_fp8(to_np_f32(x))
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)


@pytest.mark.parametrize("split", [1, 2, 4])
def test_one_hot_reads_back_weights_and_scales(split):
    n, k = 272, 512  # 3 weight row blocks (the last has 16 rows), 4 K blocks
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x38
    w[:254, 7] = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    ws = rng.integers(110, 140, size=(3, 4), dtype=np.uint8)
    cols = np.concatenate([np.arange(0, k, 5), [7, 63, 64, 127, 128, 255, 256, 511]])
    m = len(cols)
    a = np.zeros((m, k), dtype=np.uint8)
    a[np.arange(m), cols] = 0x38  # e4m3 1.0
    a_s = rng.integers(118, 136, size=(m, 4), dtype=np.uint8)  # a scale per (token, K block)
    w_d = torch.from_numpy(w).to(DEV)
    prep = L.prepare_fp8_block_weight(w_d, torch.from_numpy(ws).to(DEV))
    out = gemm(torch.from_numpy(a).to(DEV), torch.from_numpy(a_s).to(DEV), prep, split)
    raw = gemm(torch.from_numpy(a).to(DEV), torch.from_numpy(a_s).to(DEV), prep, split, raw=w_d)
    torch.cuda.synchronize()
    assert torch.equal(raw, out)
    wd = O.dequant_fp8_block(w, ws)                                    # W * 2^(ew-127), exact
    sa = O.decode_e8m0(a_s)[np.arange(m), cols // 128]                 # the scale of the K block read
    want = O.bf16_round((wd[:, cols] * sa[None, :]).T) + np.float32(0.0)
    np.testing.assert_array_equal(to_np_f32(out).view(np.uint32), want.astype(np.float32).view(np.uint32))


def run(m, n, k, *, split=None, seed=3, rows=None):
    print(f"[block fp8] gemm M={m} N={n} K={k} split={split}", flush=True)
    codes, scales = S.make_fp8_block_linear(n, k, seed=seed, device=DEV)
    x = torch.randn((m, k), device=DEV, generator=torch.Generator(DEV).manual_seed(seed + 100)).to(torch.bfloat16)
    q, s = quant(x)
    prep = L.prepare_fp8_block_weight(codes, scales)
    out = gemm(q, s, prep, split)
    raw = gemm(q, s, prep, split, raw=codes)
    torch.cuda.synchronize()
    assert torch.equal(raw, out), "checkpoint-layout and tiled weights differ"
    rows = np.arange(m) if rows is None else rows
    ref = O.block_fp8_gemm_f32(q.cpu().numpy()[rows], s.cpu().numpy()[rows], codes.cpu().numpy(),
                               scales.cpu().numpy())
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"block fp8 M={m} N={n} split={split}")
    print(f"    {err}", flush=True)


@pytest.mark.parametrize("n", [4096, 1024, 16384])
@pytest.mark.parametrize("m", [1, 64])
def test_decode_shapes(m, n):
    run(m, n, 4096)


@pytest.mark.parametrize("n", [4096, 1024, 16384])
def test_prefill_shapes_row_subset(n):
    rows = np.sort(np.random.default_rng(n).choice(8192, 96, replace=False))
    run(8192, n, 4096, rows=rows)


@pytest.mark.parametrize("split", [1, 2, 4, 8])
def test_every_split(split):
    run(64, 1024, 4096, split=split)


@pytest.mark.parametrize("m", [2, 17, 65, 129])
@pytest.mark.parametrize("n,k", [(48, 256), (208, 384), (1040, 1024)])
def test_ragged_shapes(m, n, k):
    run(m, n, k)
    run(m, n, k, split=2)


def test_reference_api_round_trip():
    """The reference's call sequence: plans, activation_quant_into into
    float8 / e8m0 tensors, block_fp8_gemm_into with the checkpoint weight
    (raw and prepared give the same bits)."""

    m, n, k = 40, 384, 1024
    print("[block fp8] reference API", flush=True)
    codes, scales = S.make_fp8_block_linear(n, k, seed=8, device=DEV)
    w = codes.view(torch.float8_e4m3fn)
    w_s = scales.view(torch.float8_e8m0fnu)
    x = S.make_hidden(m, k, seed=9, device=DEV)
    qp = F.make_quantization_plan(m, k)
    aq = torch.empty(qp.quantized_shape, dtype=F.FP8_DTYPE, device=DEV)
    a_s = torch.empty(qp.scale_shape, dtype=F.E8M0_DTYPE, device=DEV)
    F.activation_quant_into(x, aq, a_s, plan=qp)
    outs = []
    for split in (None, 2):
        gp = F.make_gemm_plan(m, n, k, split_k=split)
        ws = torch.empty(gp.workspace_shape, dtype=torch.float32, device=DEV)
        for weight in (w, L.prepare_fp8_block_weight(w, w_s)):
            out = torch.empty(gp.output_shape, dtype=torch.bfloat16, device=DEV)
            F.block_fp8_gemm_into(aq, a_s, weight, w_s, out, ws, plan=gp)
            outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[2], outs[3])
    # beside a prepared weight only its own scale tensor is accepted (no value compare)
    with pytest.raises(ValueError, match="prepared"):
        F.block_fp8_gemm_into(aq, a_s, L.prepare_fp8_block_weight(w, w_s), w_s.clone(), outs[3], ws, plan=gp)
    ref = O.block_fp8_gemm_f32(aq.view(torch.uint8).cpu().numpy(), a_s.view(torch.uint8).cpu().numpy(),
                               codes.cpu().numpy(), scales.cpu().numpy())
    for out in (outs[0], outs[2]):
        assert_moe_close(to_np_f32(out), ref, what="reference API")


@pytest.mark.parametrize("split", [2, 8])
def test_prefill_kernel_with_explicit_split(split):
    """The 8-wavefront prefill kernel over a K split (partials reduced in split order)."""

    rows = np.sort(np.random.default_rng(split).choice(8192, 64, replace=False))
    run(8192, 4096, 4096, split=split, rows=rows)


@pytest.mark.parametrize("m,n,k,split", [(1, 4096, 4096, 8), (2, 1024, 4096, 4), (4, 16384, 1024, 2),
                                         (7, 1024, 4096, 8), (16, 16384, 4096, 4), (3, 4096, 4096, 2),
                                         (5, 208, 640, 2), (9, 208, 1024, 4)])
def test_in_workgroup_split_matches_two_launch_reduction(m, n, k, split):
    """Up to 16 tokens a K split runs inside one workgroup (each wavefront
    one split's K blocks, the partials summed through LDS in split order);
    from 17 tokens the split workgroups write partials that a reduce launch
    sums.  Rows of C depend only on their row of A and the split boundaries
    are the same, so the first m rows of a 40-token call with the same split
    must carry the same bits.  Up to 4 tokens with splits covering K
    exactly the activation rows go through LDS (M=1..4 here, rows of 4, 8
    and 16 blocks); ragged N (N=208: the last 128-row scale block partial)
    and a last split with fewer blocks (K=640: 5 blocks over 2 splits of 3)
    included."""

    print(f"[block fp8] in-workgroup split M={m} N={n} K={k} split={split}", flush=True)
    codes, scales = S.make_fp8_block_linear(n, k, seed=41, device=DEV)
    prep = L.prepare_fp8_block_weight(codes, scales)
    x = torch.randn((40, k), device=DEV, generator=torch.Generator(DEV).manual_seed(m + 100 * split))
    q, s = quant(x.to(torch.bfloat16))
    small = gemm(q[:m].contiguous(), s[:m].contiguous(), prep, split)
    small_raw = gemm(q[:m].contiguous(), s[:m].contiguous(), prep, split, raw=codes)
    big = gemm(q, s, prep, split)
    torch.cuda.synchronize()
    assert torch.equal(small.view(torch.int16), small_raw.view(torch.int16))
    assert torch.equal(small.view(torch.int16), big[:m].view(torch.int16))


@pytest.mark.parametrize("m,n", [(4196, 4096), (8192, 1024)])
def test_gemm256_kernel_matches_three_stage_kernel_bits(m, n):
    """Grids of at least 256 workgroups of 256 tokens without a K split run
    the 256-token two-stage kernel: 256 channels per workgroup where that
    fills the GPU (M=4196, N=4096: 17 x 16 tiles, the last token tile
    ragged), else 128 (M=8192, N=1024: 32 x 8); smaller grids run the
    128 x 256 three-stage kernel.  A row of C depends only on its row of A,
    and both kernels add the same scaled MFMAs in K-block order, so the
    first 2048 rows and the last 100 equal a 2048-token and a 100-token
    call (split 1) bit for bit, for tiled and row-major weights; a row
    subset against the closed form as well."""

    k = 4096
    print(f"[block fp8] 256-token kernel M={m} N={n} K={k}", flush=True)
    codes, scales = S.make_fp8_block_linear(n, k, seed=51, device=DEV)
    prep = L.prepare_fp8_block_weight(codes, scales)
    x = torch.randn((m, k), device=DEV, generator=torch.Generator(DEV).manual_seed(52)).to(torch.bfloat16)
    q, s = quant(x)
    big = gemm(q, s, prep, 1)
    big_raw = gemm(q, s, prep, 1, raw=codes)
    head = gemm(q[:2048].contiguous(), s[:2048].contiguous(), prep, 1)
    tail = gemm(q[m - 100:].contiguous(), s[m - 100:].contiguous(), prep, 1)
    torch.cuda.synchronize()
    assert torch.equal(big.view(torch.int16), big_raw.view(torch.int16))
    assert torch.equal(big[:2048].view(torch.int16), head.view(torch.int16))
    assert torch.equal(big[m - 100:].view(torch.int16), tail.view(torch.int16))
    rows = np.r_[0, 255, 256, 2047, 3000, 4095, m - 100, m - 1]
    ref = O.block_fp8_gemm_f32(q.cpu().numpy()[rows], s.cpu().numpy()[rows], codes.cpu().numpy(),
                               scales.cpu().numpy())
    assert_moe_close(to_np_f32(big)[rows], ref, what=f"256-token kernel N={n}")
