"""The allocation-free fused layer entry (``dsv4moe_layer_w4a16_noalloc``)
against the existing entry (``dsv4moe_layer_w4a16`` with a caller
workspace), both called through the C ABI: identical routing, alignment and
output bits on two calls in a row, the second with fewer tokens (the static
scratch still holds the first call's contents), and a clear rejection of a
call whose workspace would not fit the static scratch."""

import ctypes

import pytest
import torch

from gaiban_lite_amd import ResidentInt4MoEWeights, _lib, max_padded_tokens, ops, synthetic as S

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SHAPE = S.FLASH
E, H, I, K = SHAPE.experts, SHAPE.hidden, SHAPE.inter, SHAPE.topk
SCRATCH_BYTES = 64 << 20


def _buffers(t):
    bs = ops.block_size_m(t, K, E)
    cap = max_padded_tokens(t * K, E, bs)
    return {
        "bs": bs,
        "cap": cap,
        "ids": torch.empty((t, K), dtype=torch.int32, device=DEV),
        "w": torch.empty((t, K), dtype=torch.float32, device=DEV),
        "margin": torch.empty((t,), dtype=torch.float32, device=DEV),
        "sorted": torch.empty((cap,), dtype=torch.int32, device=DEV),
        "eids": torch.empty(((cap + bs - 1) // bs,), dtype=torch.int32, device=DEV),
        "ntpp": torch.empty((1,), dtype=torch.int32, device=DEV),
        "out": torch.empty((t, H), dtype=torch.bfloat16, device=DEV),
    }


def _args(res, x, logits, b):
    p = _lib.ptr
    t = x.shape[0]
    return [p(x), p(logits), None, t, H, I, E, K, _lib.SCORE_FUNCS["sigmoid"], 1.0, p(res.w13_q), p(res.w13_s),
            p(res.w2_q), p(res.w2_s), p(res.w13_r), p(res.w2_r), 1, 0.0, b["bs"], p(b["ids"]), p(b["w"]), p(b["margin"]), p(b["sorted"]),
            b["cap"], p(b["eids"]), p(b["ntpp"]), p(b["out"])]


def test_noalloc_layer_matches_workspace_entry_on_two_calls():
    w = S.make_checkpoint_experts(SHAPE, seed=5, device=DEV)
    res = ResidentInt4MoEWeights.from_checkpoint_layout(*w, experts=E, has_shared=True)
    del w
    stream = _lib.current_stream(DEV)
    for t in (64, 8):  # the second call is smaller: stale scratch from the first must not leak
        print(f"[noalloc] T={t}", flush=True)
        x = S.make_hidden(t, H, seed=40 + t, device=DEV)
        logits = S.make_logits(t, E, seed=41 + t, device=DEV)
        ref = _buffers(t)
        ws = torch.empty(ops.experts_workspace_bytes(t, K, H, I, True), dtype=torch.uint8, device=DEV)
        _lib.call("dsv4moe_layer_w4a16", *_args(res, x, logits, ref), _lib.ptr(ws), ws.numel(), stream)
        got = _buffers(t)
        _lib.call("dsv4moe_layer_w4a16_noalloc", *_args(res, x, logits, got), stream)
        torch.cuda.synchronize()
        for key in ("ids", "w", "margin", "ntpp", "out"):
            assert torch.equal(got[key], ref[key]), (t, key)
        n = int(ref["ntpp"].item())
        assert torch.equal(got["sorted"][:n], ref["sorted"][:n])
        assert torch.equal(got["eids"][:n // ref["bs"]], ref["eids"][:n // ref["bs"]])
        assert torch.isfinite(got["out"].float()).all()


def test_noalloc_layer_rejects_a_workspace_above_the_scratch():
    t = 512  # needs about 74 MB of workspace at the Flash shapes
    need = ops.experts_workspace_bytes(t, K, H, I, True)
    assert need > SCRATCH_BYTES
    x = torch.empty((t, H), dtype=torch.bfloat16, device=DEV)
    logits = torch.empty((t, E), dtype=torch.float32, device=DEV)
    b = _buffers(t)
    fake = torch.empty(16, dtype=torch.uint8, device=DEV)

    class _Res:  # weight pointers are never dereferenced: the call fails before any launch
        w13_q = w13_s = w2_q = w2_s = w13_r = w2_r = fake

    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("dsv4moe_layer_w4a16_noalloc", *_args(_Res, x, logits, b), _lib.current_stream(DEV))
    assert ctypes.sizeof(ctypes.c_void_p) == 8
