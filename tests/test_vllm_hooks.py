"""The vLLM seam installers against stand-in modules (vLLM is not installed
here), the way the reference's own tests stub vllm_ascend
(tests/test_patch_fused_moe.py:521-535, 759-882, 885-917, 1929-2181).  CPU
only: what is checked is the wiring, the fail-closed paths and the contract
fields; the kernels behind the hook run in the GPU layer tests."""

import sys
from types import ModuleType, SimpleNamespace

import pytest
import torch

from vllm_moe_offload_amd import fused_moe
from vllm_moe_offload_amd.patches import patch_fused_moe as pfm


class _Comm:
    def fused_experts(self, fused_experts_input):
        return "native"

    def _maybe_apply_moe_offload_plan(self, fused_experts_input):
        return fused_experts_input


def _fake_comm(cls):
    return SimpleNamespace(MoECommMethod=cls, FusedExpertsResult=SimpleNamespace,
                           MoEFusedExpertsInput=SimpleNamespace, MoEWeights=SimpleNamespace,
                           MoERoutingParams=SimpleNamespace, MoEOffloadParams=SimpleNamespace)


def test_comm_hook_installs_once_and_keeps_the_originals():
    cls = type("Comm", (_Comm,), {})
    orig = cls.fused_experts
    assert pfm._patch_moe_comm_method_runtime_hooks(_fake_comm(cls))
    assert cls.fused_experts._latchmoe_patch_tag == pfm.PATCH_TAG
    assert cls._maybe_apply_moe_offload_plan._latchmoe_patch_tag == pfm.PATCH_TAG
    assert cls._latchmoe_original_fused_experts is orig
    installed = cls.fused_experts
    assert pfm._patch_moe_comm_method_runtime_hooks(_fake_comm(cls))  # idempotent
    assert cls.fused_experts is installed
    assert not pfm._patch_moe_comm_method_runtime_hooks(SimpleNamespace())  # no target: no-op
    # offload off: the original method runs
    inp = SimpleNamespace(offload=SimpleNamespace(enabled=False))
    assert cls().fused_experts(inp) == "native"
    assert cls()._maybe_apply_moe_offload_plan(inp) is inp


def test_comm_hook_fails_closed_for_an_offloaded_layer_without_slots(monkeypatch):
    from vllm_moe_offload_amd.moe_offload import runtime as runtime_mod

    rt = SimpleNamespace(capture_safe_slot_weights=lambda **kw: None,
                         should_use_fixed_slot_plan_for_layer=lambda lid: lid == 7)
    monkeypatch.setattr(runtime_mod, "get_moe_offload_runtime", lambda: rt)
    cls = type("Comm2", (_Comm,), {})
    pfm._patch_moe_comm_method_runtime_hooks(_fake_comm(cls))
    inp = SimpleNamespace(offload=SimpleNamespace(enabled=True, layer_id=7))
    with pytest.raises(RuntimeError, match="refusing to capture or replay"):
        cls()._maybe_apply_moe_offload_plan(inp)


def test_with_slot_weights_carries_every_contract_field():
    """Weights become the slot bank, routing gets log2phy and P, every other
    field of the input is carried over (patch_fused_moe.py:2039-2099)."""
    marker = {k: object() for k in ("w1_bias", "w2_bias", "w1_scale", "w2_scale", "w1_scale_bias",
                                    "w2_scale_bias", "w1_offset", "w2_offset", "expert_map", "mc2_mask",
                                    "pertoken_scale", "quant", "hidden", "w", "ids")}
    inp = fused_moe.MoEFusedExpertsInput(
        hidden_states=marker["hidden"], topk_weights=marker["w"], topk_ids=marker["ids"],
        weights=fused_moe.MoEWeights(w1="old1", w2="old2", **{k: marker[k] for k in (
            "w1_bias", "w2_bias", "w1_scale", "w2_scale", "w1_scale_bias", "w2_scale_bias", "w1_offset",
            "w2_offset")}),
        routing=fused_moe.MoERoutingParams(expert_map=marker["expert_map"], global_redundant_expert_num=3,
                                           mc2_mask=marker["mc2_mask"], apply_router_weight_on_input=True,
                                           pertoken_scale=marker["pertoken_scale"]),
        quant=marker["quant"], activation="silu", need_trans=True, dynamic_eplb=True, swiglu_limit=7.0,
        offload=fused_moe.MoEOffloadParams(enabled=True, profile_only=True, layer_id=5, num_logical_experts=9,
                                           expected_device_type="cuda", step_id=11),
    )
    prepared = SimpleNamespace(w1="bank13", w2="bank2", log2phy="table", physical_expert_count=64)
    out = fused_moe.with_slot_weights(inp, prepared)
    assert (out.weights.w1, out.weights.w2) == ("bank13", "bank2")
    assert all(getattr(out.weights, k) is marker[k] for k in ("w1_bias", "w2_scale", "w2_offset"))
    r = out.routing
    assert (r.log2phy, r.physical_expert_count, r.global_redundant_expert_num) == ("table", 64, 3)
    assert r.expert_map is marker["expert_map"] and r.mc2_mask is marker["mc2_mask"]
    assert r.apply_router_weight_on_input is True and r.pertoken_scale is marker["pertoken_scale"]
    assert out.quant is marker["quant"] and out.need_trans and out.dynamic_eplb and out.swiglu_limit == 7.0
    o = out.offload
    assert (o.enabled, o.profile_only, o.layer_id, o.num_logical_experts, o.step_id) == (True, True, 5, 9, 11)
    assert fused_moe.with_slot_weights(inp, prepared, use_log2phy=False, offload_enabled=False).routing.log2phy is None


@pytest.mark.parametrize("field,value,msg", [
    ("quant", object(), "quantized"),
    ("activation", "gelu", "SwiGLU only"),
    ("swiglu_limit", 7.0, "swiglu_limit"),
    ("need_trans", True, "need_trans"),
])
def test_unsupported_contract_options_fail_closed(field, value, msg):
    inp = fused_moe.MoEFusedExpertsInput(hidden_states=None, topk_weights=None, topk_ids=None)
    setattr(inp, field, value)
    with pytest.raises(RuntimeError, match=msg):
        fused_moe.check_supported_input(inp)
    inp2 = fused_moe.MoEFusedExpertsInput(hidden_states=None, topk_weights=None, topk_ids=None,
                                          routing=fused_moe.MoERoutingParams(expert_map=torch.arange(4)))
    with pytest.raises(RuntimeError, match="expert_map"):
        fused_moe.check_supported_input(inp2)


def test_engine_args_hook_adds_the_stage_split_and_fails_closed_on_full(monkeypatch):
    monkeypatch.setenv("VLLM_ASCEND_MOE_OFFLOAD_ENABLED", "1")
    monkeypatch.setenv("VLLM_ASCEND_MOE_OFFLOAD_STAGE_SEAM", "1")
    mode = {"v": "PIECEWISE"}

    class FakeEngineArgs:
        def create_engine_config(self):
            return SimpleNamespace(compilation_config=SimpleNamespace(cudagraph_mode=mode["v"], splitting_ops=[]))

    arg_utils = SimpleNamespace(EngineArgs=FakeEngineArgs)
    assert pfm._patch_engine_args_autoconfig(arg_utils)
    hooked = FakeEngineArgs.create_engine_config
    assert pfm._patch_engine_args_autoconfig(arg_utils) and FakeEngineArgs.create_engine_config is hooked
    cfg = FakeEngineArgs().create_engine_config()
    assert "vllm::moe_offload_stage" in cfg.compilation_config.splitting_ops
    mode["v"] = "FULL"
    with pytest.raises(RuntimeError, match="PIECEWISE"):
        FakeEngineArgs().create_engine_config()


def test_select_experts_hook_returns_the_injected_topk_for_the_layer():
    from vllm_moe_offload_amd.ops.fused_moe import moe_seam_inject

    class FusedMoE:
        @staticmethod
        def select_experts(hidden_states, router_logits, top_k, **kw):
            return "native_w", "native_ids"

    class Method:
        def apply(self, layer, x, router_logits):
            return FusedMoE.select_experts(x, router_logits, 2)

    assert pfm._patch_select_experts(FusedMoE) and pfm._patch_quant_method_apply(Method)
    layer = SimpleNamespace(layer_id=-1)
    assert Method().apply(layer, None, None) == ("native_w", "native_ids")
    layer = SimpleNamespace(layer_id=13)
    moe_seam_inject.set_injected_topk(13, "w13", "ids13")
    try:
        assert Method().apply(layer, None, None) == ("w13", "ids13")
    finally:
        moe_seam_inject.clear_injected_topk(13)
    assert FusedMoE.select_experts(None, None, 2) == ("native_w", "native_ids")  # no layer context


def test_apply_patches_installs_into_stubbed_vllm_modules(monkeypatch):
    comm_mod = ModuleType("vllm.model_executor.layers.fused_moe.moe_comm_method")
    comm_mod.MoECommMethod = type("CommX", (_Comm,), {})
    layer_mod = ModuleType("vllm.model_executor.layers.fused_moe.layer")

    class FusedMoE:
        @staticmethod
        def select_experts(*a, **k):
            return None, None

    class UnquantizedFusedMoEMethod:
        def apply(self, layer, *a, **k):
            return None

        def create_weights(self, layer, *a, **k):
            return None

        def process_weights_after_loading(self, layer):
            return None

    layer_mod.FusedMoE = FusedMoE
    layer_mod.UnquantizedFusedMoEMethod = UnquantizedFusedMoEMethod
    arg_mod = ModuleType("vllm.engine.arg_utils")
    arg_mod.EngineArgs = type("EngineArgs", (), {"create_engine_config": lambda self: None})
    for name, mod in (("vllm.model_executor.layers.fused_moe.moe_comm_method", comm_mod),
                      ("vllm.model_executor.layers.fused_moe.layer", layer_mod),
                      ("vllm.engine.arg_utils", arg_mod)):
        monkeypatch.setitem(sys.modules, name, mod)
    done = pfm.apply_patches()
    assert done == {"comm_method": True, "select_experts": True, "quant_apply": True, "quant_weights": True,
                    "engine_args": True, "graph_replay_profile": False}
    assert comm_mod.MoECommMethod.fused_experts._latchmoe_patch_tag == pfm.PATCH_TAG


def test_weight_hooks_create_host_experts_and_register_after_loading(monkeypatch):
    """create_weights makes host blocks for an offloaded layer and defers to
    vLLM for others; process_weights_after_loading registers both kinds
    (patch_fused_moe.py:4537-4576, 4748-4790)."""
    from vllm_moe_offload_amd.moe_offload import runtime as runtime_mod
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig

    rt = runtime_mod.MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2, cpu_first_load=True,
                                                        pin_host_memory=False,
                                                        resident_layer_ids=frozenset({4})))
    monkeypatch.setattr(runtime_mod, "get_moe_offload_runtime", lambda: rt)
    calls = []

    class Method:
        moe = SimpleNamespace(is_act_and_mul=True, has_bias=False)

        def create_weights(self, layer, num_experts, hidden_size, isz, params_dtype, **attrs):
            calls.append(("create", layer.layer_id))
            layer.w13_weight = torch.nn.Parameter(torch.ones(num_experts, 2 * isz, hidden_size), requires_grad=False)
            layer.w2_weight = torch.nn.Parameter(torch.ones(num_experts, hidden_size, isz), requires_grad=False)

        def process_weights_after_loading(self, layer):
            calls.append(("process", layer.layer_id))

    assert pfm._patch_quant_method_weights(Method) and pfm._patch_quant_method_weights(Method)  # idempotent
    offloaded, resident = torch.nn.Module(), torch.nn.Module()
    offloaded.layer_name, resident.layer_name = "model.layers.3.mlp.experts", "model.layers.4.mlp.experts"
    m = Method()
    for layer in (offloaded, resident):
        m.create_weights(layer, 4, 3, 2, torch.float32, weight_loader=None)
    assert calls == [("create", 4)]  # the offloaded layer never reached vLLM's allocation
    assert offloaded.layer_id == 3 and offloaded.w13_weight.device.type == "cpu"
    offloaded.w13_weight.data.fill_(2.0)
    offloaded.w2_weight.data.fill_(3.0)
    for layer in (offloaded, resident):
        m.process_weights_after_loading(layer)
    assert calls == [("create", 4), ("process", 4)]  # vLLM's processing ran for the resident layer only
    assert rt.is_layer_registered(3) and not rt.is_layer_registered(4)
    assert rt.host_store.get(3, 1).w13.data_ptr() == offloaded.w13_weight[1].data_ptr()
