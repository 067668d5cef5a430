"""Host-side contract of the fixed B240 alignment (``runtime/dsv4_direct/
fixed_moe_align.py:26-234,407-421``), on the CPU: the geometry constants and
their known answers, the provider's constructor checks, identity, owned
storage and call checks, the cold allocator, the metadata / non-alias
validator with the reference's exception classes, and that the hot wrapper
refuses CPU tensors (it runs the HIP kernel only).  The layout itself is
checked on the GPU (``test_gpu_graph.py``)."""

import pytest
import torch

import oracle as O
from gaiban_lite_amd import fixed_moe_align as FA
from gaiban_lite_amd.deterministic_moe_align import DeterministicMoEAlignment, max_padded_tokens

from test_runtime_lifecycle_host import _layer

CPU = torch.device("cpu")


def test_geometry_known_answers():
    # fixed_moe_align.py:29-38: 240 x 6 routes, 256 experts, block 8
    assert FA.FIXED_NUM_ASSIGNMENTS == 1440 and FA.FIXED_SENTINEL == 1440
    assert FA.FIXED_MAX_PADDED_TOKENS == 3232 == FA.fixed_b240_max_padded_tokens()
    assert FA.FIXED_MAX_BLOCKS == 404
    assert max_padded_tokens(1440, 256, 8) == 3232 == O.max_padded_tokens(1440, 256, 8)
    assert O.marlin_block_size_m(240, 6, 256) == FA.FIXED_BLOCK_SIZE
    plan = FA.FIXED_B240_ALIGNMENT_PLAN
    assert plan.route_shape == (240, 6) and plan.max_blocks == 404 and plan.workspace_capacity == 512


def test_provider_constructor_checks():
    for bad in ((240, 16), (64,), ()):
        with pytest.raises(ValueError, match="240"):
            FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=bad, slots_per_shape=1,
                                             route_kind="learned")
    for slots in (0, -1, True, 1.0):
        with pytest.raises(ValueError, match="slots_per_shape"):
            FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=(240,), slots_per_shape=slots,
                                             route_kind="learned")
    with pytest.raises(ValueError, match="learned"):
        FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=(240,), slots_per_shape=1, route_kind="hash")


def test_provider_identity_storage_and_call_checks():
    prov = FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=[240], slots_per_shape=3,
                                            route_kind="learned")
    ident = prov.provider_identity()
    assert ident == {"provider": "direct_fixed_b240_moe_alignment", "route_kind": "learned",
                     "global_row_shapes": [240], "slots_per_shape": 3, "route_shape": [240, 6],
                     "num_experts": 256, "block_size": 8, "workspace_capacity": 512, "launch_count": 1}
    store = prov.storage_tensors()
    assert isinstance(store, tuple) and len(store) == 3
    assert len({t.untyped_storage().data_ptr() for t in store}) == 3
    assert all(t.shape == (512,) and t.dtype == torch.int32 and t.is_contiguous() for t in store)
    assert prov.resident_bytes == 3 * 512 * 4
    assert prov.storage_tensors()[0] is store[0]  # stable identity: the layer checks it
    ids = torch.zeros((240, 6), dtype=torch.int32)
    out, _ = FA.allocate_fixed_b240_alignment(ids)
    with pytest.raises(ValueError, match="block 8"):
        prov(ids, block_size=16, num_experts=256, output=out, slot=0)
    with pytest.raises(ValueError, match="block 8"):
        prov(ids, block_size=8, num_experts=384, output=out, slot=0)
    with pytest.raises(TypeError):
        prov(ids, block_size=8, num_experts=256, output=out, slot=True)
    with pytest.raises(ValueError, match="not registered"):
        prov(ids, block_size=8, num_experts=256, output=out, slot=3)
    meta = torch.zeros((240, 6), dtype=torch.int32, device="meta")
    with pytest.raises(ValueError, match="route ids"):
        prov(meta, block_size=8, num_experts=256, output=out, slot=0)
    # CPU tensors pass every check, then the GPU-only wrapper refuses them
    with pytest.raises(RuntimeError, match="GPU"):
        prov(ids, block_size=8, num_experts=256, output=out, slot=1)


def test_allocate_and_validate():
    ids = torch.zeros((240, 6), dtype=torch.int32)
    out, ws = FA.allocate_fixed_b240_alignment(ids)
    assert out.sorted_token_ids.shape == (3232,) and out.expert_ids.shape == (404,)
    assert out.num_tokens_post_padded.shape == (1,) and ws.counts_and_offsets.shape == (512,)
    assert FA.validate_fixed_b240_alignment_tensors(ids, output=out, workspace=ws) == CPU
    with pytest.raises(ValueError, match="240, 6"):
        FA.allocate_fixed_b240_alignment(torch.zeros((241, 6), dtype=torch.int32))
    with pytest.raises(TypeError, match="int32"):
        FA.allocate_fixed_b240_alignment(torch.zeros((240, 6), dtype=torch.int64))
    with pytest.raises(TypeError):
        FA.allocate_fixed_b240_alignment([[0] * 6] * 240)
    with pytest.raises(ValueError, match="contiguous"):
        FA.validate_fixed_b240_alignment_tensors(torch.zeros((6, 240), dtype=torch.int32).t(), output=out,
                                                 workspace=ws)
    with pytest.raises(TypeError, match="DeterministicMoEAlignment"):
        FA.validate_fixed_b240_alignment_tensors(ids, output=(1, 2, 3), workspace=ws)
    with pytest.raises(TypeError, match="FixedB240AlignmentWorkspace"):
        FA.validate_fixed_b240_alignment_tensors(ids, output=out, workspace=ws.counts_and_offsets)
    bad_sizes = [
        DeterministicMoEAlignment(torch.zeros(3231, dtype=torch.int32), out.expert_ids, out.num_tokens_post_padded),
        DeterministicMoEAlignment(out.sorted_token_ids, torch.zeros(404, dtype=torch.int64),
                                  out.num_tokens_post_padded),
        DeterministicMoEAlignment(out.sorted_token_ids, out.expert_ids, torch.zeros(2, dtype=torch.int32)),
    ]
    for bad in bad_sizes:
        with pytest.raises(ValueError):
            FA.validate_fixed_b240_alignment_tensors(ids, output=bad, workspace=ws)
    with pytest.raises(ValueError):
        FA.validate_fixed_b240_alignment_tensors(ids, output=out, workspace=FA.FixedB240AlignmentWorkspace(
            torch.zeros(511, dtype=torch.int32)))
    # aliasing: the workspace shares the sorted ids' storage
    big = torch.zeros(3232 + 512, dtype=torch.int32)
    aliased = DeterministicMoEAlignment(big[:3232], out.expert_ids, out.num_tokens_post_padded)
    with pytest.raises(ValueError):
        FA.validate_fixed_b240_alignment_tensors(ids, output=aliased,
                                                 workspace=FA.FixedB240AlignmentWorkspace(big[3232:]))
    with pytest.raises(RuntimeError, match="GPU"):
        FA.fixed_b240_moe_align_block8(ids, output=out, workspace=ws)


def test_provider_is_accepted_by_the_layer():
    """The layer snapshots the provider's owned storage at construction and
    binds it for capture (the CPU layer runs the host lifecycle only)."""

    prov = FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=(240,), slots_per_shape=2,
                                            route_kind="learned")
    layer = _layer(rows=(240,), slots=2, provider=prov)
    assert layer.alignment_provider is prov
    other = FA.FixedB240MoEAlignmentProvider(device=CPU, global_row_shapes=(240,), slots_per_shape=2,
                                             route_kind="learned")
    layer.reset_free_slot_completion_event(240, 0)
    with pytest.raises(ValueError, match="own alignment provider"):
        with layer.bind_alignment_provider_for_capture(other, buffer_keys=[(240, 0)]):
            pass
