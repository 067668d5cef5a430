"""Alignment kernel parity: bit-exact against the oracle's closed form (itself
pinned to the list brute force on the CPU)."""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    allocate_deterministic_moe_alignment,
    deterministic_moe_align_block_size,
)

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def gpu_align(ids_np, bs, e):
    ids = torch.from_numpy(np.ascontiguousarray(ids_np.astype(np.int32))).to(DEV)
    out = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=e)
    torch.cuda.synchronize()
    return (out.sorted_token_ids.cpu().numpy(), out.expert_ids.cpu().numpy(),
            int(out.num_tokens_post_padded.cpu()[0]))


def check(ids_np, bs, e):
    s, x, n = gpu_align(ids_np, bs, e)
    ref = O.moe_align(ids_np, bs, e)
    assert n == ref.num_tokens_post_padded
    np.testing.assert_array_equal(s, ref.sorted_token_ids)
    np.testing.assert_array_equal(x, ref.expert_ids)


def uniform_ids(rng, t, e, k):
    return np.argsort(rng.random((t, e)), axis=1)[:, :k]


@pytest.mark.parametrize("t,e,k,bs", [
    (64, 8, 2, 8), (1, 256, 6, 8), (8, 256, 6, 8), (64, 256, 6, 8), (256, 256, 6, 8),
    (512, 256, 6, 16), (1024, 256, 6, 32), (2048, 256, 6, 48), (8192, 256, 6, 64),
    (4, 256, 6, 8), (240, 256, 6, 8), (3, 1024, 16, 64), (777, 384, 8, 16), (1, 2, 1, 64),
])
def test_align_uniform(t, e, k, bs):
    rng = np.random.default_rng(t * 131 + e + bs)
    check(uniform_ids(rng, t, e, k), bs, e)


def test_align_zipf_and_degenerate():
    import gaiban_lite_amd.synthetic as S

    ids = S.zipf_ids(8192, 256, 6, device=DEV).cpu().numpy()
    check(ids, 64, 256)
    check(ids[:64], 8, 256)
    degen = np.tile(np.arange(6), (1000, 1))  # every token on experts 0..5
    check(degen, 64, 256)
    check(degen, 8, 256)


def test_align_int64_input_and_caller_output():
    rng = np.random.default_rng(2)
    ids = torch.from_numpy(uniform_ids(rng, 100, 256, 6).astype(np.int64)).to(DEV)
    out = allocate_deterministic_moe_alignment(ids, block_size=16, num_experts=256)
    res = deterministic_moe_align_block_size(ids, block_size=16, num_experts=256, output=out)
    assert res is out
    ref = O.moe_align(ids.cpu().numpy(), 16, 256)
    np.testing.assert_array_equal(out.sorted_token_ids.cpu().numpy(), ref.sorted_token_ids)


def test_align_out_of_range_id_reports_minus_one():
    ids = torch.tensor([[0, 1], [2, 300]], dtype=torch.int32, device=DEV)
    out = deterministic_moe_align_block_size(ids, block_size=8, num_experts=256)
    assert int(out.num_tokens_post_padded.cpu()[0]) == -1
