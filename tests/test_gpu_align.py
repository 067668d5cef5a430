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


def split_and_single(ids_np, bs, e, fill_ws=0xA5):
    """The workgroup-split alignment (ops.align_into with a workspace, which
    starts with arbitrary bytes) and the one-workgroup kernel on the same ids."""

    from gaiban_lite_amd import ops

    ids = torch.from_numpy(np.ascontiguousarray(ids_np.astype(np.int32))).to(DEV)
    t, k = ids.shape
    need = ops.align_workspace_bytes(t, k, e)
    assert need > 0, "case below the split threshold"
    outs = []
    for ws in (torch.full((need,), fill_ws, dtype=torch.uint8, device=DEV), None):
        out = allocate_deterministic_moe_alignment(ids, block_size=bs, num_experts=e)
        out.sorted_token_ids.fill_(-7)
        out.expert_ids.fill_(-7)
        out.num_tokens_post_padded.fill_(-7)
        ops.align_into(ids, block_size=bs, num_experts=e, sorted_token_ids=out.sorted_token_ids,
                       expert_ids=out.expert_ids, num_tokens_post_padded=out.num_tokens_post_padded, workspace=ws)
        torch.cuda.synchronize()
        outs.append((out.sorted_token_ids.cpu().numpy(), out.expert_ids.cpu().numpy(),
                     int(out.num_tokens_post_padded.cpu()[0])))
    return outs


@pytest.mark.parametrize("t,e,k,bs", [
    (1366, 256, 6, 64),     # 8196 ids: 2 chunks, the second ragged
    (1024, 256, 8, 64),     # exactly 8192 ids
    (8192, 256, 6, 64),     # the prefill benchmark: 12 chunks
    (8192, 256, 6, 128),
    (4096, 8, 2, 64),       # few experts, 2 chunks
    (1000, 1024, 16, 64),   # 1024 experts, 16000 ids
    (65536, 256, 8, 64),    # 524288 ids: capped at 64 chunks of 8192
    (9000, 2, 1, 16),
])
def test_split_align_matches_oracle_and_single_workgroup(t, e, k, bs):
    print(f"[align split] T={t} E={e} k={k} bs={bs}", flush=True)
    rng = np.random.default_rng(t + e + k + bs)
    ids = rng.integers(0, e, size=(t, k)) if k > e // 4 else uniform_ids(rng, t, e, k)
    split, single = split_and_single(ids, bs, e)
    ref = O.moe_align(ids, bs, e)
    for s, x, n in (split, single):
        assert n == ref.num_tokens_post_padded
        np.testing.assert_array_equal(s, ref.sorted_token_ids)
        np.testing.assert_array_equal(x, ref.expert_ids)


def test_split_align_zipf_and_hot_expert():
    import gaiban_lite_amd.synthetic as S

    print("[align split] zipf / one expert", flush=True)
    for ids in (S.zipf_ids(8192, 256, 6, device=DEV).cpu().numpy(),
                np.full((4096, 4), 17),                      # every id on one expert
                np.tile(np.arange(6), (2000, 1))):           # six experts, in order
        split, _ = split_and_single(ids, 64, 256)
        ref = O.moe_align(ids, 64, 256)
        assert split[2] == ref.num_tokens_post_padded
        np.testing.assert_array_equal(split[0], ref.sorted_token_ids)
        np.testing.assert_array_equal(split[1], ref.expert_ids)


@pytest.mark.parametrize("where", ["first", "last"])
def test_split_align_out_of_range_writes_only_minus_one(where):
    """An id outside [0, experts) in any chunk: num_tokens_post_padded = -1 and
    no other output element is written."""

    print(f"[align split] bad id in the {where} chunk", flush=True)
    rng = np.random.default_rng(9)
    ids = uniform_ids(rng, 4096, 256, 6)
    if where == "first":
        ids[3, 2] = 256
    else:
        ids[-1, 5] = -1
    split, single = split_and_single(ids, 64, 256)
    for s, x, n in (split, single):
        assert n == -1
        assert (s == -7).all() and (x == -7).all()
