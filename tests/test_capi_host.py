"""CPU-side checks of the C ABI library and the host logic: the library loads
and exports every function declared in include/dsv4moe.h; its host-only
policy functions equal the oracle; validation rejects bad arguments before
any launch; the Python boundary validates configs and route overrides."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from gaiban_lite_amd import _lib, ops
from gaiban_lite_amd import moe_runtime as R
from gaiban_lite_amd import synthetic as S
from gaiban_lite_amd.deterministic_moe_align import max_padded_tokens

HEADER = Path(__file__).resolve().parents[1] / "include" / "dsv4moe.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsv4moe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in dsv4moe.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.dsv4moe_abi_version() == 3


def test_host_policy_functions_match_oracle():
    lib = _lib.load()
    for rows in (1, 4, 8, 64, 100, 256, 512, 1000, 1024, 2048, 4096, 8192, 32768):
        for item in (1, 2):
            assert lib.dsv4moe_block_size_m(rows, 6, 256, item) == O.marlin_block_size_m(rows, 6, 256, item)
    for a, e, bs in ((24, 256, 8), (1440, 256, 8), (49152, 256, 64), (3, 8, 16), (7, 1024, 64)):
        assert lib.dsv4moe_max_padded_tokens(a, e, bs) == O.max_padded_tokens(a, e, bs) == max_padded_tokens(a, e, bs)
    assert lib.dsv4moe_block_size_m(0, 6, 256, 2) == -1
    assert lib.dsv4moe_max_padded_tokens(0, 256, 8) == -1


def _einval(name, *args):
    rc = getattr(_lib.load(), name)(*args)
    assert rc == _lib.DSV4MOE_EINVAL, (name, rc)
    return _lib.last_error()


def test_validation_rejects_before_launch():
    fake = ctypes.c_void_p(0x1000)
    assert "experts" in _einval("dsv4moe_route_topk", fake, None, 4, 0, 2, 0, 1.0, fake, fake, None, None, None, None)
    assert "topk" in _einval("dsv4moe_route_topk", fake, None, 4, 8, 9, 0, 1.0, fake, fake, None, None, None, None)
    assert "score_func" in _einval("dsv4moe_route_topk", fake, None, 4, 8, 2, 7, 1.0, fake, fake, None, None, None, None)
    assert "capacity" in _einval("dsv4moe_align", fake, 4, 6, 256, 8, fake, 191, fake, 24, fake, None)
    assert "multiple of 32" in _einval("dsv4moe_pack_int4_g128", fake, fake, 1, 48, 128, 0, fake, fake, None)
    assert "pairing" in _einval("dsv4moe_pack_int4_g128", fake, fake, 1, 64, 128, 2, fake, fake, None)
    assert "block_size" in _einval("dsv4moe_experts_w4a16", fake, 4, 4096, 2048, 256, 6, fake, fake, fake, fake,
                                   fake, fake, 1, fake, fake, 192, fake, fake, 12, 0.0, fake, fake, 1 << 30, None)
    assert "hidden" in _einval("dsv4moe_experts_w4a16", fake, 4, 4000, 2048, 256, 6, fake, fake, fake, fake,
                               fake, fake, 1, fake, fake, 192, fake, fake, 8, 0.0, fake, fake, 1 << 30, None)
    ws = ops.experts_workspace_bytes(4, 6, 4096, 2048, True)
    assert "workspace" in _einval("dsv4moe_experts_w4a16", fake, 4, 4096, 2048, 256, 6, fake, fake, fake, fake,
                                  fake, fake, 1, fake, fake, 192, fake, fake, 8, 0.0, fake,
                                  ctypes.c_void_p(0x100000), ws - 1, None)
    # the scale ratios of the prefill kernels are required
    good_ws = ctypes.c_void_p(0x100000)
    assert "scale-ratio" in _einval("dsv4moe_experts_w4a16", fake, 4, 4096, 2048, 256, 6, fake, fake, fake, fake,
                                    None, fake, 1, fake, fake, 192, fake, fake, 8, 0.0, fake, good_ws, ws, None)
    assert "multiple of 32" in _einval("dsv4moe_pack_int4_ratios", fake, 1, 48, 128, fake, None)
    assert "multiple of 128" in _einval("dsv4moe_pack_int4_ratios", fake, 1, 64, 100, fake, None)
    assert "null" in _einval("dsv4moe_pack_int4_ratios", None, 1, 64, 128, fake, None)


def test_align_workspace_policy_and_validation():
    """The split alignment needs [chunks][experts + 1] int32 of scratch, chunks
    of >= 4096 ids (multiples of 1024), at most 64 chunks; below 8192 ids one
    workgroup aligns and no scratch is needed."""

    lib = _lib.load()
    assert lib.dsv4moe_align_workspace_bytes(1365, 6, 256) == 0        # 8190 ids
    assert lib.dsv4moe_align_workspace_bytes(1024, 8, 256) == 2 * 257 * 4   # 8192 ids: 2 x 4096
    assert lib.dsv4moe_align_workspace_bytes(8192, 6, 256) == 12 * 257 * 4  # 49152 ids: 12 x 4096
    assert lib.dsv4moe_align_workspace_bytes(2049, 6, 8) == 4 * 9 * 4       # 12294 ids: 4 x 4096 (last ragged)
    assert lib.dsv4moe_align_workspace_bytes(1 << 20, 8, 1024) == 64 * 1025 * 4  # capped at 64 chunks
    assert lib.dsv4moe_align_workspace_bytes(0, 6, 256) == 0
    fake = ctypes.c_void_p(0x1000)
    t, k, e, bs = 8192, 6, 256, 64
    cap = O.max_padded_tokens(t * k, e, bs)
    nb = (cap + bs - 1) // bs
    need = lib.dsv4moe_align_workspace_bytes(t, k, e)
    assert "workspace" in _einval("dsv4moe_align_ws", fake, t, k, e, bs, fake, cap, fake, nb, fake,
                                  fake, need - 1, None)
    assert "workspace" in _einval("dsv4moe_align_ws", fake, t, k, e, bs, fake, cap, fake, nb, fake,
                                  None, need, None)
    assert "capacity" in _einval("dsv4moe_align_ws", fake, t, k, e, bs, fake, cap - 1, fake, nb, fake,
                                 fake, need, None)


def test_w8a16_validation_and_split_policy():
    fake = ctypes.c_void_p(0x1000)
    lib = _lib.load()
    args = lambda m, n, k, split, ws_bytes, layout=0: (fake, m, n, k, fake, layout, fake, split, fake, ws_bytes,
                                                       fake, None)
    assert "multiple of 16" in _einval("dsv4moe_w8a16_linear", *args(4, 40, 4096, 1, 0))
    assert "multiple of 128" in _einval("dsv4moe_w8a16_linear", *args(4, 64, 4000, 1, 0))
    assert "split_k" in _einval("dsv4moe_w8a16_linear", *args(4, 64, 4096, 3, 1 << 30))
    assert "K-block" in _einval("dsv4moe_w8a16_linear", *args(4, 64, 256, 4, 1 << 30))
    need = lib.dsv4moe_w8a16_workspace_bytes(4, 64, 2)
    assert need == 2 * 4 * 64 * 4 and lib.dsv4moe_w8a16_workspace_bytes(4, 64, 1) == 0
    assert "workspace" in _einval("dsv4moe_w8a16_linear", *args(4, 64, 4096, 2, need - 1))
    assert "weight_layout" in _einval("dsv4moe_w8a16_linear", *args(4, 64, 4096, 1, 0, layout=2))
    assert "weight_layout" in _einval("dsv4moe_w8a16_fp8_linear", *args(4, 64, 4096, 1, 0, layout=-1))
    assert "multiple of 16" in _einval("dsv4moe_pack_int8", fake, 24, 128, fake, None)
    for layout in (_lib.WEIGHT_TILED, _lib.WEIGHT_ROWMAJOR):
        assert lib.dsv4moe_w8a16_linear(fake, 0, 64, 4096, fake, layout, fake, 1, None, 0, fake,
                                        None) == _lib.DSV4MOE_OK
    # this library's policy: a power of two in [1, 8] leaving >= 4 windows of 64 K per split;
    # up to 16 tokens (the split inside the workgroup) 4, or 8 from N = 8192; above, raised only
    # while the grid is below 512 workgroups
    for m in (1, 16, 17, 64, 65, 8192):
        for n in (1024, 4096, 16384):
            split = lib.dsv4moe_w8a16_split_k(m, n, 4096)
            assert split in (1, 2, 4, 8)
            assert 4096 // 64 // split >= 4
            if m <= 16:
                assert split == (8 if n >= 8192 else 4)
    assert lib.dsv4moe_w8a16_split_k(1, 4096, 512) == 2  # 8 windows: 2 splits of 4
    assert lib.dsv4moe_w8a16_split_k(8192, 4096, 4096) == 1
    assert lib.dsv4moe_w8a16_split_k(0, 4096, 4096) == -1


def test_block_fp8_validation_and_split_policy():
    fake = ctypes.c_void_p(0x1000)
    lib = _lib.load()
    g = lambda m, n, k, split, ws, layout=0: (fake, fake, m, n, k, fake, layout, fake, split, fake, ws, fake, None)
    assert "multiple of 16" in _einval("dsv4moe_block_fp8_gemm", *g(4, 40, 4096, 1, 0))
    assert "multiple of 128" in _einval("dsv4moe_block_fp8_gemm", *g(4, 64, 4000, 1, 0))
    assert "split_k" in _einval("dsv4moe_block_fp8_gemm", *g(4, 64, 4096, 16, 1 << 30))
    assert "K-block" in _einval("dsv4moe_block_fp8_gemm", *g(4, 64, 256, 4, 1 << 30))
    need = lib.dsv4moe_block_fp8_workspace_bytes(4, 64, 2)
    assert need == 2 * 4 * 64 * 4 and lib.dsv4moe_block_fp8_workspace_bytes(4, 64, 1) == 0
    assert "workspace" in _einval("dsv4moe_block_fp8_gemm", *g(4, 64, 4096, 2, need - 1))
    assert "weight_layout" in _einval("dsv4moe_block_fp8_gemm", *g(4, 64, 4096, 1, 0, layout=7))
    assert "x_dtype" in _einval("dsv4moe_act_quant_block_fp8", fake, 3, 4, 128, fake, fake, None)
    assert "multiple of 128" in _einval("dsv4moe_act_quant_block_fp8", fake, 0, 4, 100, fake, fake, None)
    assert lib.dsv4moe_block_fp8_gemm(*g(0, 64, 4096, 1, 0)) == _lib.DSV4MOE_OK
    # this library's split: a power of two in [1, 8] leaving >= 2 K blocks per split; up to 16
    # tokens 4, or 8 from N = 8192; above, raised only while the grid is below 512 workgroups
    for m in (1, 16, 17, 64, 65, 8192):
        for n in (1024, 4096, 16384):
            split = lib.dsv4moe_block_fp8_split_k(m, n, 4096)
            assert split in (1, 2, 4, 8) and 32 // split >= 2
            if m <= 16:
                assert split == (8 if n >= 8192 else 4)
    assert lib.dsv4moe_block_fp8_split_k(1, 16384, 512) == 2  # 4 K blocks: 2 splits of 2
    assert lib.dsv4moe_block_fp8_split_k(8192, 4096, 4096) == 1
    assert lib.dsv4moe_block_fp8_split_k(0, 4096, 4096) == -1


def test_block_fp8_plans_mirror_reference_contract():
    from gaiban_lite_amd import fp8_linear as F

    qp = F.make_quantization_plan(33, 512)
    assert qp.quantized_shape == (33, 512) and qp.scale_shape == (33, 4) and qp.grid == (3, 4)
    gp = F.make_gemm_plan(64, 1024, 4096, split_k=4)
    assert gp.workspace_shape == (4, 64, 1024) and gp.workspace_bytes == 4 * 64 * 1024 * 4
    assert gp.weight_scale_shape == (8, 32) and gp.k_blocks_per_split == 8 and gp.dispatch == "split_k_reduce"
    assert F.make_gemm_plan(8192, 4096, 4096).split_k == 1
    for bad in (dict(split_k=3), dict(split_k=16), dict(split_k=True)):
        with pytest.raises(ValueError):
            F.make_gemm_plan(64, 1024, 4096, **bad)
    with pytest.raises(ValueError):
        F.make_gemm_plan(64, 1024, 4000)
    with pytest.raises(ValueError):
        F.make_quantization_plan(4, 256, block_m=3)
    assert F.primitive_contract()["supported_split_k"] == [1, 2, 4, 8]


@pytest.mark.parametrize("module", ["fp8_linear", "weight_only_linear"])
def test_gemm_plans_reject_unsupported_tuning_and_n(module):
    """The reference's tuning checks (``weight_only_linear.py:147-165``): each
    field must be one of its supported values and block_n must divide the
    128-channel scale block; N values the HIP kernels cannot run (not a
    multiple of 16) are refused when the plan is built, not at launch."""

    import importlib

    M = importlib.import_module(f"gaiban_lite_amd.{module}")
    from gaiban_lite_amd.linear_plan import GemmTuning

    for ok in (GemmTuning(), GemmTuning(16, 128, 8, 2), GemmTuning(64, 32, 4, 4)):
        assert M.make_gemm_plan(64, 1024, 4096, tuning=ok).tuning == ok
    for bad in (GemmTuning(block_m=48), GemmTuning(block_m=128), GemmTuning(block_n=256), GemmTuning(block_n=16),
                GemmTuning(num_warps=2), GemmTuning(num_warps=16), GemmTuning(num_stages=1),
                GemmTuning(num_stages=5), GemmTuning(block_m=True), GemmTuning(block_n=64.0)):
        with pytest.raises(ValueError, match="tuning"):
            M.make_gemm_plan(64, 1024, 4096, tuning=bad)
    with pytest.raises(TypeError):
        M.make_gemm_plan(64, 1024, 4096, tuning=(32, 64, 4, 3))
    for n in (1000, 24, 1):
        with pytest.raises(ValueError, match="multiple of 16"):
            M.make_gemm_plan(64, n, 4096)
    assert M.make_gemm_plan(64, 48, 4096).n == 48


def test_workspace_formula():
    # x row sums (per 64 columns) + h + h row sums + fp32 contributions, each 256-byte aligned
    t, k, h, i = 64, 6, 4096, 2048
    rows = t * k + t

    def a(v):
        return (v + 255) // 256 * 256

    expect = a(4 * t * (h // 64)) + a(2 * rows * i) + a(4 * rows * (i // 64)) + a(4 * rows * h)
    assert ops.experts_workspace_bytes(t, k, h, i, True) == expect


def test_config_validation():
    R.FLASH_CONFIG.validate()
    with pytest.raises(ValueError):
        R.TP4MoEConfig(world_size=4).validate()
    with pytest.raises(ValueError):
        R.TP4MoEConfig(hidden_size=4000).validate()
    with pytest.raises(ValueError):
        R.TP4MoEConfig(topk=17, experts=256).validate()
    with pytest.raises(ValueError):
        R.TP4MoEConfig(score_func="relu").validate()
    with pytest.raises(ValueError):
        R.TP4MoEConfig(clamp_limit=-1.0).validate()
    with pytest.raises(ValueError):
        R.ResidentGateWeights(weight=torch.zeros(4, 4), bias=torch.zeros(4), tid2eid=torch.zeros(2, 2, dtype=torch.int64))


def test_route_override_validation_cpu():
    cfg = R.TP4MoEConfig(experts=8, topk=2, route_scale=1.5, hidden_size=128, intermediate_size=128)
    cpu = torch.device("cpu")
    ids = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    w = torch.tensor([[0.75, 0.75], [1.0, 0.5]], dtype=torch.float32)
    got_ids, got_w = R._snapshot_route_override(R.MoERouteOverride(ids, w), rows=2, config=cfg, device=cpu)
    assert torch.equal(got_ids, ids) and got_ids.data_ptr() != ids.data_ptr()
    bad = [
        (torch.tensor([[0, 0], [2, 3]], dtype=torch.int32), w, "same expert twice"),
        (torch.tensor([[0, 9], [2, 3]], dtype=torch.int32), w, "outside"),
        (ids, torch.tensor([[0.7, 0.7], [1.0, 0.5]]), "sum to 1.5"),
        (ids, torch.tensor([[1.5, 0.0], [1.0, 0.5]]), "strictly positive"),
        (ids.long(), w, "int32"),
    ]
    for i, ww, msg in bad:
        with pytest.raises(TypeError if i.dtype != torch.int32 else ValueError, match=msg):
            R._snapshot_route_override(R.MoERouteOverride(i, ww), rows=2, config=cfg, device=cpu)


def test_synthetic_generators_are_seeded():
    a = S.make_checkpoint_experts(S.TINY, seed=3, device="cpu", experts=range(2, 4))
    b = S.make_checkpoint_experts(S.TINY, seed=3, device="cpu")
    assert torch.equal(a[0][0], b[0][2]) and torch.equal(a[3][1], b[3][3])
    s = a[1].float()
    assert float(s.min()) >= 0.0049 and float(s.max()) <= 0.0201
    ids = S.zipf_ids(8192, 256, 6, device="cpu")
    counts = np.bincount(ids.numpy().reshape(-1), minlength=256)
    assert counts.max() / counts.mean() > 10  # heavy skew (hottest expert >> mean)


def test_w8a16_fp8_validation_and_e8m0_preflight():
    from gaiban_lite_amd import weight_only_linear as L

    fake = ctypes.c_void_p(0x1000)
    args = lambda m, n, k, split, ws_bytes, layout=0: (fake, m, n, k, fake, layout, fake, split, fake, ws_bytes,
                                                       fake, None)
    assert "multiple of 16" in _einval("dsv4moe_w8a16_fp8_linear", *args(4, 40, 4096, 1, 0))
    assert "multiple of 128" in _einval("dsv4moe_w8a16_fp8_linear", *args(4, 64, 4000, 1, 0))
    assert "k must be <= 32768" in _einval("dsv4moe_w8a16_fp8_linear", *args(4, 64, 32896, 1, 0))
    assert "null" in _einval("dsv4moe_w8a16_fp8_linear", fake, 4, 64, 4096, None, 0, fake, 1, None, 0, fake, None)
    assert _lib.load().dsv4moe_w8a16_fp8_linear(fake, 0, 64, 4096, fake, 1, fake, 1, None, 0, fake,
                                                None) == _lib.DSV4MOE_OK
    # the reference's cold preflight: the reserved E8M0 byte 255 is rejected at load time
    codes = torch.zeros((128, 256), dtype=torch.uint8)
    bad = torch.tensor([[127, 255]], dtype=torch.uint8)
    with pytest.raises(ValueError, match="255"):
        L.prepare_fp8_block_weight(codes, bad)
    with pytest.raises(TypeError, match="scale"):
        L.prepare_fp8_block_weight(codes, torch.zeros((1, 1), dtype=torch.uint8))


def test_block_fp8_mirror_rejects_host_tensors_and_bad_dtypes():
    """The fp8_linear mirror validates like the reference module before any
    launch: device placement, dtypes, shapes, and the reserved E8M0 byte."""

    from gaiban_lite_amd import fp8_linear as F

    qp = F.make_quantization_plan(4, 256)
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device"):
        F.activation_quant_into(x, torch.empty(4, 256, dtype=F.FP8_DTYPE), torch.empty(4, 2, dtype=F.E8M0_DTYPE),
                                plan=qp)
    gp = F.make_gemm_plan(4, 64, 256, split_k=1)
    with pytest.raises(ValueError, match="device"):
        F.block_fp8_gemm_into(torch.empty(4, 256, dtype=F.FP8_DTYPE), torch.empty(4, 2, dtype=F.E8M0_DTYPE),
                              torch.empty(64, 256, dtype=F.FP8_DTYPE), torch.empty(1, 2, dtype=F.E8M0_DTYPE),
                              torch.empty(4, 64, dtype=torch.bfloat16), torch.empty(0), plan=gp)
    bad = torch.full((2, 2), 255, dtype=torch.uint8).view(torch.float8_e8m0fnu)
    with pytest.raises(ValueError, match="255"):
        F.validate_e8m0_scale_values("w_scale", bad)
    with pytest.raises(TypeError):
        F.validate_e8m0_scale_values("w_scale", torch.zeros(2, 2, dtype=torch.uint8))
