"""Plugin entry point, custom-op schemas and the splitting-op contract
(reference tests/test_plugin_contract.py:43-79 and the op ABI of
moe_router_op.py:128-162, moe_offload_stage_op.py:523-529)."""

import types

import pytest
import torch


def test_register_is_idempotent_and_registers_seam_ops():
    import vllm_moe_offload_amd

    vllm_moe_offload_amd.register()
    vllm_moe_offload_amd.register()
    for name in ("moe_router", "moe_router_indirect", "moe_offload_stage", "moe_mlp", "moe_mlp_shared"):
        assert hasattr(torch.ops.vllm, name), name
    schema = str(torch.ops.vllm.moe_offload_stage.default._schema)
    assert "Tensor(a0!) topk_ids" in schema and "-> ()" in schema
    assert "Tensor(a0!) hidden_states" in str(torch.ops.vllm.moe_mlp.default._schema)


def test_router_fake_impl_abi():
    from vllm_moe_offload_amd.ops.fused_moe.moe_router_op import _moe_router_fake

    h = torch.empty(5, 16, dtype=torch.bfloat16)
    w, ids = _moe_router_fake(h, torch.empty(5, 8), 2, False, True, None, None, "softmax", 1.0, None, 8)
    assert w.shape == (5, 2) and w.dtype == torch.bfloat16 and ids.dtype == torch.int32
    w, ids = _moe_router_fake(h, torch.empty(5, 8), 2, False, True, None, None, "softmax", 1.0, None, 8, True, 1)
    assert w.shape == (5, 3) and ids.shape == (5, 3)


def test_entry_point_declared():
    import tomli
    from pathlib import Path

    data = tomli.loads((Path(__file__).resolve().parents[1] / "vllm-ascend-hust-latchmoe_amd" / "pyproject.toml").read_text())
    assert data["project"]["entry-points"]["vllm.general_plugins"]["moe_offload_ascend"] == "vllm_moe_offload_amd:register"


def test_splitting_op_contract_fails_closed_on_full_graphs():
    from vllm_moe_offload_amd.plugin import STAGE_SPLITTING_OP, ensure_moe_offload_splitting_op

    cfg = types.SimpleNamespace(cudagraph_mode=types.SimpleNamespace(name="PIECEWISE"), splitting_ops=["vllm::unified_attention"])
    ensure_moe_offload_splitting_op(cfg)
    assert STAGE_SPLITTING_OP in cfg.splitting_ops
    with pytest.raises(RuntimeError, match="PIECEWISE"):
        ensure_moe_offload_splitting_op(types.SimpleNamespace(cudagraph_mode=types.SimpleNamespace(name="FULL"), splitting_ops=[]))


def test_stage_op_is_a_noop_during_capture_and_in_regime_a(monkeypatch):
    from vllm_moe_offload_amd.moe_offload import runtime as rtm
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, _moe_offload_stage_impl

    rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=8))
    try:
        # regime A: slots >= experts, nothing is staged per step
        _moe_offload_stage_impl(torch.tensor([[0, 1]], dtype=torch.int32), 3, 4, PHASE_DECODE)
        monkeypatch.setattr(rtm, "_is_current_graph_capturing", lambda: True)
        rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2))
        with pytest.raises(RuntimeError, match="unregistered fixed-slot MoE layer"):
            _moe_offload_stage_impl(torch.tensor([[0, 1]], dtype=torch.int32), 3, 4, PHASE_DECODE)
    finally:
        rtm.reset_moe_offload_runtime()


def test_stage_op_stages_or_defers_overflow_to_waves():
    from vllm_moe_offload_amd.moe_offload import runtime as rtm
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, PHASE_PREFILL, _moe_offload_stage_impl

    class L(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer_id = 3
            self.w13_weight = torch.nn.Parameter(torch.zeros(6, 2, 1))
            self.w2_weight = torch.nn.Parameter(torch.zeros(6, 1, 1))

    rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2, b2_wave_prefill=True))
    try:
        rt = rtm._runtime
        rt.register_layer_for_fixed_slots(L(), slot_device=torch.device("cpu"))
        ids = torch.tensor([[4, 1]], dtype=torch.int32)
        _moe_offload_stage_impl(ids, 3, 6, PHASE_DECODE)
        assert rt.log2phy_buffer(3).tolist() == [-1, 0, -1, -1, 1, -1]
        big = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
        _moe_offload_stage_impl(big, 3, 6, PHASE_PREFILL)
        assert rt.log2phy_buffer(3).tolist() == [-1, 0, -1, -1, 1, -1]  # deferred, untouched
        assert rt.consume_prefill_route_stats(layer_id=3, topk_ids=big) == {0: 1, 1: 1, 2: 1, 3: 1}
    finally:
        rtm.reset_moe_offload_runtime()


def test_stage_op_stages_a_decode_overflow_pass_instead_of_waves():
    from vllm_moe_offload_amd.moe_offload import runtime as rtm
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, PHASE_PREFILL, _moe_offload_stage_impl

    class L(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer_id = 3
            self.w13_weight = torch.nn.Parameter(torch.arange(12.0).reshape(6, 2, 1))
            self.w2_weight = torch.nn.Parameter(torch.arange(6.0).reshape(6, 1, 1))

    rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2, b2_wave_prefill=True,
                                                          decode_overflow=True))
    try:
        rt = rtm._runtime
        rt.register_layer_for_fixed_slots(L(), slot_device=torch.device("cpu"))
        ids = torch.tensor([[0, 1], [2, 1], [3, 1]], dtype=torch.int32)  # 4 experts, 2 slots
        _moe_offload_stage_impl(ids, 3, 6, PHASE_DECODE)
        main, ovf = rt.log2phy_buffer(3).tolist(), rt.decode_overflow_slot_weights(layer_id=3).log2phy.tolist()
        assert rt.consume_prefill_route_stats(layer_id=3, topk_ids=ids) is None  # not deferred
        assert [e for e in range(6) if main[e] >= 0] == [0, 1]  # expert 1 (3 tokens) first, then id order
        assert [e for e in range(6) if ovf[e] >= 0] == [2, 3]
        # a prefill-phase overflow still goes to the waves
        _moe_offload_stage_impl(ids, 3, 6, PHASE_PREFILL)
        assert rt.consume_prefill_route_stats(layer_id=3, topk_ids=ids) == {0: 1, 1: 3, 2: 1, 3: 1}
    finally:
        rtm.reset_moe_offload_runtime()


def test_stage_op_stages_a_regime_a_layer_whose_full_residency_was_not_staged():
    """Slots >= experts without graph mode: nothing staged the table at
    registration, so the seam stages per step instead of leaving the pairs
    unmapped."""
    from vllm_moe_offload_amd.moe_offload import runtime as rtm
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, _moe_offload_stage_impl

    class L(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer_id = 3
            self.w13_weight = torch.nn.Parameter(torch.zeros(4, 2, 1))
            self.w2_weight = torch.nn.Parameter(torch.zeros(4, 1, 1))

    for graph_mode in (False, True):
        rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=4,
                                                              graph_compatible_offload=graph_mode))
        try:
            rt = rtm._runtime
            rt.register_layer_for_fixed_slots(L(), slot_device=torch.device("cpu"))
            assert rt.stage_full_residency_slot_plan(layer_id=3) is graph_mode
            _moe_offload_stage_impl(torch.tensor([[2, 1]], dtype=torch.int32), 3, 4, PHASE_DECODE)
            table = rt.log2phy_buffer(3).tolist()
            assert table[1] >= 0 and table[2] >= 0
            if graph_mode:
                assert table == [0, 1, 2, 3]  # the static table, untouched by the seam
        finally:
            rtm.reset_moe_offload_runtime()


def test_stage_op_fails_closed_on_ids_outside_the_layer():
    """An id outside [0, total) has no slot, stage buffer or wave: the seam
    raises on the host copy of the ids instead of letting a pass skip it."""
    from vllm_moe_offload_amd.moe_offload import runtime as rtm
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, PHASE_PREFILL, _moe_offload_stage_impl

    class L(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer_id = 3
            self.w13_weight = torch.nn.Parameter(torch.zeros(6, 2, 1))
            self.w2_weight = torch.nn.Parameter(torch.zeros(6, 1, 1))

    rtm._runtime = rtm.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2, b2_wave_prefill=True,
                                                          decode_overflow=True))
    try:
        rt = rtm._runtime
        rt.register_layer_for_fixed_slots(L(), slot_device=torch.device("cpu"))
        before = rt.log2phy_buffer(3).tolist()
        for bad, phase in (([[0, 6]], PHASE_DECODE), ([[-1, 1]], PHASE_DECODE), ([[0, 1], [2, 7]], PHASE_PREFILL)):
            with pytest.raises(RuntimeError, match="outside"):
                _moe_offload_stage_impl(torch.tensor(bad, dtype=torch.int32), 3, 6, phase)
        assert rt.log2phy_buffer(3).tolist() == before  # nothing staged
        _moe_offload_stage_impl(torch.tensor([[0, 5]], dtype=torch.int32), 3, 6, PHASE_DECODE)  # in range
    finally:
        rtm.reset_moe_offload_runtime()
