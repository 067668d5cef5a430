"""Host-side lifecycle of the ``TP4MoE`` drop-in, on the CPU: route-capture
registration and snapshots (``moe_runtime.py:1017-1227``), the alignment
provider's capture binding (``:825-978``), slot leases, and argument checks
that must fail before any launch (hash token ids outside the table, the
reserved E8M0 scale byte).  A layer built on the CPU runs no kernels: every
call raises after the host checks."""

import pytest
import torch

from gaiban_lite_amd import (
    MoERouteCaptureBuffer,
    MoERouteCaptureEvidence,
    ResidentGateWeights,
    ResidentInt4MoEWeights,
    ResidentMXFP4MoEWeights,
    TP4MoE,
    TP4MoEConfig,
)
from gaiban_lite_amd.deterministic_moe_align import DeterministicMoEAlignment

E, H, I, K = 8, 256, 256, 2
CPU = torch.device("cpu")


def _resident():
    e = E + 1
    return ResidentInt4MoEWeights(
        w13_q=torch.zeros((e, I * H), dtype=torch.uint8), w13_s=torch.ones((e, 2 * I * H // 128), dtype=torch.bfloat16),
        w2_q=torch.zeros((e, H * I // 2), dtype=torch.uint8), w2_s=torch.ones((e, H * I // 128), dtype=torch.bfloat16),
        experts=E, hidden_size=H, intermediate_size=I, has_shared=True)


class _Provider:
    """A minimal alignment provider with owned storage."""

    def __init__(self):
        self.store = (torch.zeros(64, dtype=torch.int32),)

    def storage_tensors(self):
        return self.store

    def __call__(self, ids, *, block_size, num_experts, output: DeterministicMoEAlignment, slot):
        return output


def _layer(rows=(4, 16), slots=2, provider=None, tid2eid=None):
    cfg = TP4MoEConfig(hidden_size=H, intermediate_size=I, experts=E, topk=K, route_scale=1.0, clamp_limit=0.0,
                       score_func="sigmoid", shared_experts=1)
    gate = ResidentGateWeights(weight=torch.zeros((E, H), dtype=torch.bfloat16), tid2eid=tid2eid)
    return TP4MoE(config=cfg, resident=_resident(), gate=gate, device=CPU, global_row_shapes=rows,
                  slots_per_shape=slots, alignment_provider=provider)


def test_register_route_capture_contract():
    layer = _layer()
    cap = layer.register_route_capture(4, 1)
    assert isinstance(cap, MoERouteCaptureBuffer)
    assert cap.ids.shape == (4, K) and cap.ids.dtype == torch.int32 and bool((cap.ids == -1).all())
    assert cap.weights.dtype == torch.float32 and cap.generation.dtype == torch.int64
    assert layer.registered_route_capture_slots == {4: (1,)}
    assert layer.route_capture_buffer(4, 1) is cap
    with pytest.raises(RuntimeError, match="already registered"):
        layer.register_route_capture(4, 1)
    with pytest.raises(TypeError):
        layer.register_route_capture(True, 0)
    with pytest.raises(ValueError, match="no registered buffers"):
        layer.register_route_capture(5, 0)
    with pytest.raises(ValueError, match="no route capture"):
        layer.route_capture_buffer(16, 0)
    # a capture whose tensor was swapped is refused
    forged = MoERouteCaptureBuffer(global_rows=4, slot=1, owner_id=id(layer), ids=cap.ids.clone(),
                                   weights=cap.weights, generation=cap.generation,
                                   tensor_pointers=cap.tensor_pointers)
    layer._route_captures[(4, 1)] = forged
    with pytest.raises(ValueError):
        layer.route_capture_buffer(4, 1)


def test_snapshot_route_capture_generations():
    layer = _layer()
    cap = layer.register_route_capture(16, 0)
    with pytest.raises(ValueError, match="positive integer"):
        layer.snapshot_route_capture(16, 0, expected_generation=0)
    with pytest.raises(ValueError, match="positive integer"):
        layer.snapshot_route_capture(16, 0, expected_generation=True)
    with pytest.raises(RuntimeError, match="not recorded"):
        layer.snapshot_route_capture(16, 0, expected_generation=1)
    # what a call's capture step does (on the current stream): copy and bump
    ids = torch.arange(16 * K, dtype=torch.int32).view(16, K) % E
    w = torch.full((16, K), 0.5)
    got_w, got_ids = layer._capture_route((16, 0), w, ids)
    assert got_ids is cap.ids and got_w is cap.weights and int(cap.generation) == 1
    with pytest.raises(RuntimeError, match="expected 2"):
        layer.snapshot_route_capture(16, 0, expected_generation=2)
    ev = layer.snapshot_route_capture(16, 0, expected_generation=1)
    assert isinstance(ev, MoERouteCaptureEvidence)
    assert torch.equal(ev.ids, ids) and torch.equal(ev.weights, w) and ev.generation == 1
    assert ev.ids.data_ptr() != cap.ids.data_ptr() and len(ev.route_digest) == 64
    with pytest.raises(ValueError, match="already lives"):
        layer._capture_route((16, 0), cap.weights, cap.ids)
    layer.reset_route_capture_generation(16, 0)
    assert int(cap.generation) == 0


def test_capture_binding_lease_and_lifecycle():
    provider = _Provider()
    layer = _layer(provider=provider)
    with pytest.raises(ValueError, match="own alignment provider"):
        with layer.bind_alignment_provider_for_capture(_Provider(), buffer_keys=[(4, 0)]):
            pass
    with pytest.raises(ValueError, match="at least one"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[]):
            pass
    with pytest.raises(TypeError):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(4, True)]):
            pass
    with pytest.raises(ValueError, match="not a registered"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(5, 0)]):
            pass
    with pytest.raises(ValueError, match="unique"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(4, 0), (4, 0)]):
            pass
    layer._buffers[(4, 0)].has_completion_event = True
    with pytest.raises(RuntimeError, match="reset the completion events"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(4, 0)]):
            pass
    layer.reset_free_slot_completion_event(4, 0)
    layer._buffers[(16, 1)].state = "in_flight"
    with pytest.raises(RuntimeError, match="every slot free"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(4, 0)]):
            pass
    layer._buffers[(16, 1)].state = "free"
    # the lease: None selects the built-in alignment; other slots are refused; no nesting
    with pytest.raises(KeyError):
        with layer.bind_alignment_provider_for_capture(None, buffer_keys=[(4, 0)]):
            assert layer._active_alignment_provider is None
            with pytest.raises(RuntimeError, match="nested"):
                with layer.bind_alignment_provider_for_capture(None, buffer_keys=[(4, 1)]):
                    pass
            with pytest.raises(RuntimeError, match="outside the active graph-capture binding"):
                layer(torch.zeros((1, 16, H), dtype=torch.bfloat16))
            with pytest.raises(RuntimeError, match="during a capture binding"):
                layer.reset_free_slot_completion_event(4, 1)
            with pytest.raises(RuntimeError, match="during a capture binding"):
                layer.register_route_capture(4, 0)
            raise KeyError("capture failed")  # a failed capture that left every slot unchanged
    assert layer._active_alignment_provider is provider and not layer._alignment_provider_poisoned
    # a "capture" that never ran the listed slot leaves it without a completion event: poisoned
    with pytest.raises(RuntimeError, match="inconsistent"):
        with layer.bind_alignment_provider_for_capture(provider, buffer_keys=[(4, 0)]):
            pass
    assert layer._alignment_provider_poisoned
    with pytest.raises(RuntimeError, match="poisoned"):
        layer.reset_free_slot_completion_event(4, 0)
    with pytest.raises(RuntimeError, match="poisoned"):
        layer.register_route_capture(16, 0)


def test_cpu_layer_refuses_to_compute():
    layer = _layer()
    with pytest.raises(ValueError, match="computes on a GPU"):
        layer(torch.zeros((1, 4, H), dtype=torch.bfloat16))
    assert layer.slot_completion_status(4, 0) == {"state": "free", "has_completion_event": False}


def test_hash_token_ids_outside_the_table_are_rejected():
    table = torch.stack([torch.arange(K) + i % (E - K) for i in range(100)]).to(torch.int64)
    layer = _layer(tid2eid=table)
    assert layer.check_hash_token_ids is False  # opt-in: one host read per call
    layer.check_hash_token_ids = True
    x = torch.zeros((1, 4, H), dtype=torch.bfloat16)
    for bad in ([[0, 1, 100, 2]], [[-1, 0, 0, 0]]):
        with pytest.raises(ValueError, match=r"input_ids_local: values span .* outside \[0, 100\)"):
            layer(x, input_ids_local=torch.tensor(bad, dtype=torch.int64))
    assert layer.slot_completion_status(4, 0)["state"] == "free"


def test_mxfp4_residents_reject_the_reserved_scale_byte():
    e = 2
    w13 = torch.zeros((e, 2 * I, H // 2), dtype=torch.uint8)
    w2 = torch.zeros((e, H, I // 2), dtype=torch.uint8)
    s13 = torch.full((e, 2 * I, H // 32), 120, dtype=torch.uint8)
    s2 = torch.full((e, H, I // 32), 120, dtype=torch.uint8)
    s2[1, 3, 4] = 255
    with pytest.raises(ValueError, match="255"):
        ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13, w2, s2, experts=1, has_shared=True)
    s13[0, 0, 0] = 255
    with pytest.raises(ValueError, match="w13_scale"):
        ResidentMXFP4MoEWeights.from_checkpoint_layout(w13, s13.view(torch.float8_e8m0fnu), w2, s2, experts=1,
                                                       has_shared=True)
