"""W4A8 path on the fp8 MFMA: the per-row e4m3 quantiser bit for bit against
the oracle (codes, scales) and its group sums; the grouped experts against
the fp32 W4A8 oracle ``moe_w4a8_f32`` (quantised activations, dequantised
int4 weights, fp32 accumulation) to max_rel and rel_fro <= 1e-2, on the tiny
layer, the Flash decode layer (uniform and Zipf routing) and Flash prefill
row subsets; and the TP4MoE drop-in with ``marlin_input_dtype=float8_e4m3fn``.
"""

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import (
    ResidentGateWeights,
    ResidentInt4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    ops,
    route_from_logits,
    synthetic as S,
)
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size
from helpers import DeviceExpertSource, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
PERM = np.array([0, 4, 1, 5, 2, 6, 3, 7])
_LAYERS: dict = {}


def natural_order(q: np.ndarray) -> np.ndarray:
    """Undo the MFMA byte order of dsv4moe_act_quant_fp8."""

    rows, k = q.shape
    g = k // 128
    out = np.empty_like(q)
    src = q.reshape(rows, g, 4, 4, 8)  # group, j, d, byte
    dst = out.reshape(rows, g, 4, 4, 8)  # group, d, j, k-offset   (k = 32d + 8j + off)
    for b in range(8):
        dst[:, :, :, :, PERM[b]] = src[:, :, :, :, b].transpose(0, 1, 3, 2)
    return out


@pytest.mark.parametrize("rows,k,scale", [(64, 4096, 1.0), (7, 512, 1e-3), (130, 2048, 300.0)])
def test_act_quant_bit_exact(rows, k, scale):
    g = torch.Generator(DEV).manual_seed(rows + k)
    x = (torch.randn((rows, k), device=DEV, generator=g) * scale).to(torch.bfloat16)
    x[0, :7] = 0.0
    q = torch.empty((rows, k), dtype=torch.uint8, device=DEV)
    s = torch.empty((rows,), dtype=torch.float32, device=DEV)
    gs = torch.empty((rows, k // 128), dtype=torch.float32, device=DEV)
    ops.act_quant_fp8_into(x, q, s, gs)
    torch.cuda.synchronize()
    ref_q, ref_s = O.act_quant_per_token_fp8(to_np_f32(x))
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), ref_s.reshape(-1).view(np.uint32))
    codes = natural_order(q.cpu().numpy())
    np.testing.assert_array_equal(codes, O.fp8_e4m3_encode(ref_q))
    ref_sums = ref_q.astype(np.float64).reshape(rows, -1, 128).sum(axis=2)
    np.testing.assert_allclose(gs.cpu().numpy(), ref_sums, rtol=1e-5, atol=1e-3)


def test_act_quant_zero_row():
    x = torch.zeros((4, 512), dtype=torch.bfloat16, device=DEV)
    q = torch.empty((4, 512), dtype=torch.uint8, device=DEV)
    s = torch.empty((4,), dtype=torch.float32, device=DEV)
    gs = torch.empty((4, 4), dtype=torch.float32, device=DEV)
    ops.act_quant_fp8_into(x, q, s, gs)
    torch.cuda.synchronize()
    assert np.all(s.cpu().numpy() == np.float32(1e-12) / np.float32(448.0))
    assert not q.cpu().numpy().any() and not gs.cpu().numpy().any()


def layer(shape: S.LayerShape, seed: int = 0):
    key = (shape, seed)
    if key not in _LAYERS:
        if len(_LAYERS) >= 2:
            _LAYERS.clear()
            torch.cuda.empty_cache()
        w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=seed, device=DEV)
        res = ResidentInt4MoEWeights.from_checkpoint_layout(
            w13, s13, w2, s2, experts=shape.experts, has_shared=shape.has_shared,
            marlin_input_dtype=torch.float8_e4m3fn)
        _LAYERS[key] = (res, DeviceExpertSource(w13, s13, w2, s2))
    return _LAYERS[key]


def check(shape, t, *, rows=None, clamp=0.0, zipf=False, block_size=None, seed=1):
    print(f"[w4a8] E={shape.experts} H={shape.hidden} I={shape.inter} k={shape.topk} T={t} zipf={zipf} "
          f"clamp={clamp} bs={block_size}", flush=True)
    res, src = layer(shape)
    x = S.make_hidden(t, shape.hidden, seed=seed, device=DEV)
    logits = S.make_logits(t, shape.experts, seed=seed + 1, device=DEV)
    r = route_from_logits(logits, topk=shape.topk, score_func="sigmoid")
    ids, w = r.routing_ids, r.routing_weights
    if zipf:
        ids = S.zipf_ids(t, shape.experts, shape.topk, seed=4, device=DEV)
    bs = block_size or ops.block_size_m(t, shape.topk, shape.experts, 1)
    align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=shape.experts)
    out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.experts_w4a8_workspace_bytes(t, shape.topk, shape.hidden, shape.inter, shape.has_shared),
                     dtype=torch.uint8, device=DEV)
    ops.experts_w4a8_into(
        x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, experts=shape.experts,
        inter=shape.inter, has_shared=shape.has_shared, route_weights=w,
        sorted_token_ids=align.sorted_token_ids, expert_ids=align.expert_ids,
        num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs, clamp_limit=clamp,
        out=out, workspace=ws)
    torch.cuda.synchronize()
    rows = np.arange(t) if rows is None else np.asarray(rows)
    ref = O.moe_w4a8_f32(to_np_f32(x), ids.cpu().numpy(), w.cpu().numpy(), src,
                         shared_index=shape.experts if shape.has_shared else None,
                         clamp_limit=clamp, rows=rows)
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"w4a8 T={t}")
    print(f"    {err}", flush=True)


TINY_SHARED = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)


@pytest.mark.parametrize("bs", [8, 16, 32, 48, 64])
def test_tiny_every_block_size(bs):
    check(TINY_SHARED, 64, block_size=bs)


def test_tiny_no_shared_and_clamp():
    check(S.TINY, 64)
    check(TINY_SHARED, 37, clamp=0.5)


def test_flash_decode_uniform():
    check(S.FLASH, 64)


def test_flash_decode_zipf():
    check(S.FLASH, 64, zipf=True)


def test_flash_prefill_subset():
    rows = np.sort(np.random.default_rng(7).choice(2048, 48, replace=False))
    check(S.FLASH, 2048, rows=rows)


def test_flash_prefill_zipf_subset():
    rows = np.sort(np.random.default_rng(8).choice(8192, 32, replace=False))
    check(S.FLASH, 8192, rows=rows, zipf=True)


def test_extreme_scale_spread():
    """Gate rows whose group scales alternate 2^100 / 2^-100 (beyond any
    running-sum ratio in fp32) and a 2^40 spread in w2: the W4A8 kernels
    scale every group exactly, so the prefill output (blocks of 64) equals
    the decode kernels' (blocks of 16) and the fp32 W4A8 oracle."""

    shape = TINY_SHARED
    print("[w4a8] extreme scale spread", flush=True)
    w13, s13, w2, s2 = S.make_checkpoint_experts(shape, seed=31, device=DEV)
    g = torch.arange(s13.shape[-1], device=DEV)
    wild = torch.where(g % 2 == 0, torch.tensor(2.0 ** 100, device=DEV), torch.tensor(2.0 ** -100, device=DEV))
    s13[3, :shape.inter] = (wild * 1e-2).to(torch.bfloat16)
    s2[5] = (s2[5].float() * torch.where(torch.arange(s2.shape[-1], device=DEV) % 2 == 0, 2.0 ** 20,
                                        2.0 ** -20)).to(torch.bfloat16)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts, has_shared=True,
                                                        marlin_input_dtype=torch.float8_e4m3fn)
    src = DeviceExpertSource(w13, s13, w2, s2)
    t = 256
    x = S.make_hidden(t, shape.hidden, seed=32, device=DEV)
    ids = torch.stack([torch.full((t,), 3, device=DEV), (torch.arange(t, device=DEV) % 7 + 4) % 8], dim=1)
    ids[::5, 1] = 5
    ids = ids.to(torch.int32)
    w = torch.full((t, 2), 0.5, device=DEV, dtype=torch.float32)
    outs = {}
    for bs in (16, 64):
        align = deterministic_moe_align_block_size(ids, block_size=bs, num_experts=shape.experts)
        out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(ops.experts_w4a8_workspace_bytes(t, 2, shape.hidden, shape.inter, True),
                         dtype=torch.uint8, device=DEV)
        ops.experts_w4a8_into(
            x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, experts=shape.experts,
            inter=shape.inter, has_shared=True, route_weights=w, sorted_token_ids=align.sorted_token_ids,
            expert_ids=align.expert_ids, num_tokens_post_padded=align.num_tokens_post_padded, block_size=bs,
            clamp_limit=0.0, out=out, workspace=ws)
        torch.cuda.synchronize()
        outs[bs] = to_np_f32(out)
        assert np.isfinite(outs[bs]).all(), bs
    ref = O.moe_w4a8_f32(to_np_f32(x), ids.cpu().numpy(), w.cpu().numpy(), src, shared_index=shape.experts)
    assert np.abs(ref).max() > 1e25  # the 2^100 groups dominate
    assert_moe_close(outs[64], outs[16], what="prefill vs decode")
    assert_moe_close(outs[64], ref, what="prefill vs oracle")
    assert_moe_close(outs[16], ref, what="decode vs oracle")


def test_layer_w4a8_dropin():
    res, src = layer(TINY_SHARED)
    cfg = TP4MoEConfig(hidden_size=1024, intermediate_size=512, experts=8, topk=2, route_scale=1.0,
                       clamp_limit=0.0, score_func="sigmoid", shared_experts=1)
    gate = ResidentGateWeights(weight=torch.zeros(8, 1024, dtype=torch.bfloat16, device=DEV))
    m = TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[64],
               marlin_input_dtype=torch.float8_e4m3fn)
    assert m.block_size_for(64) >= 16  # 1-byte activations floor the block size at 16
    x = S.make_hidden(64, 1024, seed=21, device=DEV)
    logits = S.make_logits(64, 8, seed=22, device=DEV)
    out, trace = m(x.view(1, 64, 1024), router_logits=logits)
    torch.cuda.synchronize()
    ref_route = O.route_topk(logits.cpu().numpy(), 2, score_func=O.SCORE_SIGMOID)
    assert trace.route_ids_row_zero == tuple(int(v) for v in ref_route.ids[0])
    ref = O.moe_w4a8_f32(to_np_f32(x), ref_route.ids, ref_route.weights, src, shared_index=8)
    assert_moe_close(to_np_f32(out.view(64, -1)), ref, what="layer w4a8")
    with pytest.raises(ValueError):
        TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[64])  # dtype mismatch
