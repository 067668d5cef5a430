"""W4A8 over the checkpoint's MXFP4 experts -- the reference's W4A8 mode on
its routed-expert format: ``_fused_marlin_moe(input_dtype=float8_e4m3fn)``
over MXFP4 weights with the ``is_a_8bit`` repack (``runtime/dsv4_direct/ops/
marlin_moe.py:197-222``, ``moe_runtime.py:207-235``) -- on gfx950's
block-scaled fp8 x fp4 MFMA:

* the W4A8 packer equals an independent numpy statement of its lane layout
  (lane L: the 16 checkpoint bytes of row L%16, K 128g + 32(L/16) ..);
* the grouped experts equal ``moe_w4a8_mxfp4_f32`` (per-token e4m3 x and h,
  exactly dequantised weights, fp32 accumulation) to max_rel and rel_fro <=
  1e-2: the tiny layer at every block size (decode and prefill kernels),
  E8M0 scales drawn per 32-K group from 2^-40 .. 2^10 and the edge bytes 0
  (2^-127) / 127 / 135 (a wrong lane-to-scale-group mapping fails), Flash
  T=64 and T=8192 with uniform and Zipf routing;
* the TP4MoE drop-in with ``marlin_input_dtype=float8_e4m3fn`` over
  ``ResidentMXFP4MoEWeights``, and the reference loader
  ``load_resident_moe_layer`` feeding it from a safetensors checkpoint.
"""

import numpy as np
import pytest
import torch

import oracle as O
from checkpoint_fixture import write_checkpoint
from gaiban_lite_amd import (
    ResidentGateWeights,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
    checkpoint as CK,
    ops,
    route_from_logits,
    synthetic as S,
)
from gaiban_lite_amd.deterministic_moe_align import deterministic_moe_align_block_size
from helpers import DeviceMXFP4Source, assert_moe_close, to_np_f32

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
FP8 = torch.float8_e4m3fn
SMALL = S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=True)
_LAYERS: dict = {}


def np_tile_pack_w4a8(canon: np.ndarray, gated: bool) -> np.ndarray:
    """Independent numpy statement of the W4A8 MXFP4 tile layout."""

    n, half_k = canon.shape
    groups = half_k * 2 // 128
    lane = np.arange(64)

    def row0(p, m):
        return (p * 16 + m * (n // 2)) if gated else ((2 * p + m) * 16)

    out = np.zeros((n // 32, groups, 2, 64, 16), dtype=np.uint8)
    for p in range(n // 32):
        for m in range(2):
            rows = row0(p, m) + lane % 16
            for g in range(groups):
                b0 = 64 * g + 16 * (lane // 16)
                for b in range(16):
                    out[p, g, m, :, b] = canon[rows, b0 + b]
    return out.reshape(-1)


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("n,k,batch", [(32, 128, 1), (64, 512, 2)])
def test_pack_w4a8_layout(n, k, batch, gated):
    g = torch.Generator(DEV).manual_seed(n + k + gated)
    canon = torch.randint(0, 256, (batch, n, k // 2), dtype=torch.uint8, device=DEV, generator=g)
    scales = torch.randint(100, 140, (batch, n, k // 32), dtype=torch.uint8, device=DEV, generator=g)
    q, s = ops.pack_mxfp4_g32(canon, scales, gated=gated, w4a8=True)
    _, s_ref = ops.pack_mxfp4_g32(canon, scales, gated=gated)
    torch.cuda.synchronize()
    for b in range(batch):
        np.testing.assert_array_equal(q[b].cpu().numpy(), np_tile_pack_w4a8(canon[b].cpu().numpy(), gated))
    assert torch.equal(s, s_ref)  # the scale layout is the W4A16 MXFP4 one


def layer(shape, seed=0, scale_fn=None):
    key = (shape, seed, scale_fn)
    if key not in _LAYERS:
        if len(_LAYERS) >= 2:
            _LAYERS.clear()
            torch.cuda.empty_cache()
        w13, s13, w2, s2 = S.make_checkpoint_experts_mxfp4(shape, seed=seed, device=DEV)
        if scale_fn is not None:
            s13, s2 = scale_fn(s13), scale_fn(s2)
        res = ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=shape.experts,
                                                              has_shared=shape.has_shared, marlin_input_dtype=FP8)
        _LAYERS[key] = (res, DeviceMXFP4Source(w13, s13, w2, s2))
    return _LAYERS[key]


def check(shape, t, *, rows=None, block_size=None, clamp=0.0, seed=1, ids=None, scale_fn=None, stagewise=False):
    print(f"[w4a8 mxfp4] E={shape.experts} H={shape.hidden} I={shape.inter} k={shape.topk} T={t} "
          f"bs={block_size} zipf={ids is not None}", flush=True)
    res, src = layer(shape, scale_fn=scale_fn)
    x = S.make_hidden(t, shape.hidden, seed=seed, device=DEV)
    r = route_from_logits(S.make_logits(t, shape.experts, seed=seed + 1, device=DEV), topk=shape.topk)
    route_ids = r.routing_ids if ids is None else ids
    bs = block_size or ops.block_size_m(t, shape.topk, shape.experts, 1)
    a = deterministic_moe_align_block_size(route_ids, block_size=bs, num_experts=shape.experts)
    out = torch.empty((t, shape.hidden), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.experts_w4a8_workspace_bytes(t, shape.topk, shape.hidden, shape.inter, shape.has_shared),
                     dtype=torch.uint8, device=DEV)
    ops.experts_w4a8_mxfp4_into(
        x, w13q=res.w13_q, w13s=res.w13_s, w2q=res.w2_q, w2s=res.w2_s, experts=shape.experts,
        inter=shape.inter, has_shared=shape.has_shared, route_weights=r.routing_weights,
        sorted_token_ids=a.sorted_token_ids, expert_ids=a.expert_ids,
        num_tokens_post_padded=a.num_tokens_post_padded, block_size=bs, clamp_limit=clamp,
        out=out, workspace=ws)
    torch.cuda.synchronize()
    if stagewise:
        _check_stages(shape, t, x, route_ids, r.routing_weights, src, ws, out)
        return out
    rows = np.arange(t) if rows is None else np.asarray(rows)
    ref = O.moe_w4a8_mxfp4_f32(to_np_f32(x), route_ids.cpu().numpy(), r.routing_weights.cpu().numpy(), src,
                               shared_index=shape.experts if shape.has_shared else None, clamp_limit=clamp,
                               rows=rows)
    err = assert_moe_close(to_np_f32(out)[rows], ref, what=f"w4a8 mxfp4 T={t} bs={bs}")
    print(f"    {err}", flush=True)
    return out


def _check_stages(shape, t, x, ids, weights, src, ws, out):
    """Each GEMM against the oracle on its own inputs: h (bf16, before its
    e4m3 quantisation) against the oracle's stage 1 on the quantised x, and
    the output against the oracle's stage 2 on the kernel's own e4m3 h codes
    and row scales.  With widely spread scales the whole pipeline is
    ill-conditioned -- one h value rounding to the neighbouring bf16 flips
    its e4m3 code (or its row's scale), which a large weight scale then
    carries into the output -- so the stages are held to the bar
    separately."""

    k, e, i = shape.topk, shape.experts, shape.inter
    v = ops.w4a8_workspace_views(ws, t, k, shape.hidden, i, shape.has_shared)
    ids, weights = ids.cpu().numpy(), weights.cpu().numpy()
    xq, xs = O.act_quant_per_token_fp8(to_np_f32(x))
    xd = (xq * xs).astype(np.float32)
    pairs = [(tok * k + j, tok, int(ids[tok, j]), float(weights[tok, j])) for tok in range(t) for j in range(k)]
    if shape.has_shared:
        pairs += [(t * k + tok, tok, e, 1.0) for tok in range(t)]
    h_ref = np.zeros((len(pairs), i), dtype=np.float32)
    for row, tok, ex, _ in pairs:
        w13 = src.w13(ex)
        h_ref[row] = O.bf16_round(O.swiglu_f32(xd[tok:tok + 1] @ w13[:i].T, xd[tok:tok + 1] @ w13[i:].T, 0.0))[0]
    assert_moe_close(to_np_f32(v["h"]), h_ref, what=f"stage 1 h T={t}")
    hq = O.fp8_e4m3_decode(v["hq"].cpu().numpy()) * v["hscale"].cpu().numpy()[:, None]
    y = np.zeros((t, shape.hidden), dtype=np.float64)
    for row, tok, ex, w in pairs:
        y[tok] += (hq[row] @ src.w2(ex).T.astype(np.float64)) * w
    assert_moe_close(to_np_f32(out), y, what=f"stage 2 T={t}")


@pytest.mark.parametrize("bs", [16, 32, 48, 64])
def test_every_block_size(bs):
    check(SMALL, 64, block_size=bs)


def test_small_decode_clamp_and_no_shared():
    check(SMALL, 8, clamp=0.5)
    check(S.LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=False), 37, block_size=16)


def _spread(s):
    # one E8M0 byte per 32-K group, 2^-6 .. 2^6, independent per group: a
    # lane applying another group's byte is off by up to 2^12.  (A much wider
    # spread makes the W4A8 result itself ill-conditioned: one h code moving
    # by an e4m3 step under a 2^10 scale then dominates an output.)
    g = torch.Generator(DEV).manual_seed(int(s.numel()) % 1000)
    return torch.randint(121, 134, s.shape, dtype=torch.uint8, device=DEV, generator=g)


def _edges(s):
    table = torch.tensor([0, 100, 127, 135], dtype=torch.uint8, device=DEV)
    g = torch.Generator(DEV).manual_seed(3)
    return table[torch.randint(0, 4, s.shape, device=DEV, generator=g)]


@pytest.mark.parametrize("kind", ["spread", "edges"])
@pytest.mark.parametrize("t,bs", [(64, 16), (200, 64)])
def test_scales_per_32k_group(t, bs, kind):
    """Each 32-K group carries its own power of two, so every lane of the
    MFMA must apply its own group's scale byte; the edge bytes include 0
    (2^-127, the reference's E8M0 decode of byte 0)."""

    check(SMALL, t, block_size=bs, seed=5, scale_fn=_spread if kind == "spread" else _edges,
          stagewise=kind == "spread")


def test_flash_decode_uniform():
    check(S.FLASH, 64, clamp=10.0)


def test_flash_decode_zipf():
    check(S.FLASH, 64, ids=S.zipf_ids(64, 256, 6, device=DEV))


def test_flash_prefill_8192_uniform_subset():
    rows = np.sort(np.random.default_rng(21).choice(8192, 24, replace=False))
    check(S.FLASH, 8192, rows=np.r_[0, rows, 8191], seed=13)


def test_flash_prefill_8192_zipf_subset():
    ids = S.zipf_ids(8192, 256, 6, device=DEV)
    hot = int(torch.argmax(torch.bincount(ids.flatten(), minlength=256)))
    hot_rows = torch.nonzero((ids == hot).any(dim=1)).flatten()[[0, -1]].cpu().numpy()
    check(S.FLASH, 8192, rows=np.r_[0, 4097, 8191, hot_rows], seed=17, ids=ids)


def test_tp4moe_dropin_and_reference_loader(tmp_path):
    """``load_resident_moe_layer`` with the reference's keywords and a
    SHA-256 checkpoint id, ``marlin_input_dtype=float8_e4m3fn``: the routed
    experts packed for the W4A8 kernels, the FP8 shared expert, the learned
    gate; the layer equals the W4A8 oracle on the raw checkpoint values plus
    the shared expert's bf16 path."""

    E, H, I = 8, 512, 1024
    print("[w4a8 mxfp4] loader + drop-in", flush=True)
    raw = write_checkpoint(tmp_path, layer_id=3, experts=E, hidden=H, inter=I, seed=12)
    sha = "0123456789abcdef" * 4
    res = CK.load_resident_moe_layer(stage_root=tmp_path, layer_id=3, rank=0, world_size=1, hidden_size=H,
                                     intermediate_size=I, n_experts=E, device=DEV, checkpoint_id=sha,
                                     marlin_input_dtype=FP8)
    assert res.marlin_input_dtype is FP8 and res.checkpoint_id == sha and res.layer_id == 3
    assert (res.rank, res.world_size, res.intermediate_start, res.intermediate_end) == (0, 1, 0, I)
    assert res.routed is res and res.shared is res.shared_fp8 is not None
    gate = CK.load_gate(stage_root=tmp_path, layer_id=3, experts=E, hidden_size=H, device=DEV, checkpoint_id=sha)
    cfg = TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=2, route_scale=1.5, clamp_limit=10.0,
                       score_func="sqrtsoftplus", shared_experts=1)
    layer_ = TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[64, 256],
                    marlin_input_dtype=FP8)
    assert layer_.block_size_for(64) >= 16
    p = "layers.3.ffn"
    w13 = torch.stack([torch.cat([raw[f"{p}.experts.{e}.w1.weight"], raw[f"{p}.experts.{e}.w3.weight"]])
                       for e in range(E)]).view(torch.uint8).numpy()
    s13 = torch.stack([torch.cat([raw[f"{p}.experts.{e}.w1.scale"], raw[f"{p}.experts.{e}.w3.scale"]])
                       for e in range(E)]).view(torch.uint8).numpy()
    w2 = torch.stack([raw[f"{p}.experts.{e}.w2.weight"] for e in range(E)]).view(torch.uint8).numpy()
    s2 = torch.stack([raw[f"{p}.experts.{e}.w2.scale"] for e in range(E)]).view(torch.uint8).numpy()
    src = O.MXFP4ExpertSource(w13, s13, w2, s2)
    sp = f"{p}.shared_experts"
    sh = [raw[k].contiguous().view(torch.uint8).numpy() for k in
          (f"{sp}.w1.weight", f"{sp}.w1.scale", f"{sp}.w3.weight", f"{sp}.w3.scale", f"{sp}.w2.weight",
           f"{sp}.w2.scale")]
    for t in (64, 256):
        x = S.make_hidden(t, H, seed=30 + t, device=DEV)
        lg = S.make_logits(t, E, seed=31 + t, device=DEV)
        out = layer_.forward_tensor(x.view(1, t, H), router_logits=lg)
        torch.cuda.synchronize()
        r = O.route_topk(lg.cpu().numpy(), 2, score_func=O.SCORE_SQRTSOFTPLUS, bias=raw[f"{p}.gate.bias"].numpy(),
                         route_scale=1.5)
        xf = to_np_f32(x)
        routed = O.bf16_round(O.moe_w4a8_mxfp4_f32(xf, r.ids, r.weights, src, clamp_limit=10.0))
        want = O.bf16_round(routed + O.shared_fp8_bf16(xf, *sh, 10.0))
        assert_moe_close(to_np_f32(out.view(t, H)), want, what=f"w4a8 mxfp4 layer T={t}")
    with pytest.raises(ValueError):  # the resident was packed for W4A8
        TP4MoE(config=cfg, resident=res, gate=gate, device=DEV, global_row_shapes=[64])
