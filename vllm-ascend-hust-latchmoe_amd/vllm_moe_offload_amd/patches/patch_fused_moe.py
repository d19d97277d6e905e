"""Installs the slot-bank fused-MoE seam into a vLLM process.

Three hooks, each idempotent (a tag on the installed function), each a no-op
when its target is absent:

  * the fused-experts extension hook: a MoECommMethod class (the seam the
    reference patches) gets fused_experts / _maybe_apply_moe_offload_plan
    that, for an offloaded layer, swap the expert weights for the layer's
    address-stable slot bank and run the gfx950 kernels; other layers keep
    the original methods;
  * the router hook: a select_experts function or method returns the top-k
    the router piece injected for the current layer (moe_seam_inject) and,
    for offloaded layers, calls the stage op on the ids it computes, so the
    PIECEWISE graph splits there; the layer context comes from the quant
    method's apply();
  * EngineArgs.create_engine_config: after vLLM builds its config, the
    compilation config must be PIECEWISE with vllm::moe_offload_stage among
    the splitting ops (added when missing; FULL modes fail closed).

apply_patches() looks the targets up in the installed vLLM and installs what
it finds.  The reference installs the same three on vLLM-Ascend:
patches/patch_fused_moe.py:1959-4042 (_patch_moe_comm_method_runtime_hooks),
:4509-4870 (select_experts / apply), :5409-5443
(_patch_engine_args_autoconfig).
"""

from __future__ import annotations

import importlib
import os
import threading
from contextlib import contextmanager

import torch

PATCH_TAG = "vllm_moe_offload_amd.moe_comm_method_runtime"
SELECT_TAG = "vllm_moe_offload_amd.select_experts"
ENGINE_TAG = "vllm_moe_offload_amd.engine_args"
WEIGHTS_TAG = "vllm_moe_offload_amd.cpu_first_weights"
REPLAY_TAG = "vllm_moe_offload_amd.graph_replay_profile"

# the quant method's apply() publishes its layer here for select_experts
_layer_ctx = threading.local()


def _tagged(fn, tag: str):
    fn._latchmoe_patch_tag = tag
    return fn


def _is_tagged(fn, tag: str) -> bool:
    return getattr(fn, "_latchmoe_patch_tag", None) == tag


def _contract(comm, name: str, fallback):
    """A contract class from the seam module, vLLM's runtime-args module, or
    this build's stand-in."""
    found = getattr(comm, name, None)
    if found is not None:
        return found
    for mod in ("vllm.model_executor.layers.fused_moe.moe_runtime_args",
                "vllm_ascend.ops.fused_moe.moe_runtime_args"):
        try:
            found = getattr(importlib.import_module(mod), name, None)
        except Exception:
            found = None
        if found is not None:
            return found
    return fallback


def _graph_capture_slot_weights(runtime, *, layer_id: int):
    """Capture-safe slot weights of a layer; an offloaded layer without them
    fails closed (its native weights are gone)."""
    prepared = runtime.capture_safe_slot_weights(layer_id=int(layer_id))
    if prepared is None and runtime.should_use_fixed_slot_plan_for_layer(int(layer_id)):
        raise RuntimeError(
            f"fixed-slot MoE layer {int(layer_id)} has no registered slot bank; refusing to capture or replay "
            "the native expert weights"
        )
    return prepared


def _patch_moe_comm_method_runtime_hooks(_comm) -> bool:
    """Install the slot-bank fused_experts / _maybe_apply_moe_offload_plan on
    _comm.MoECommMethod.  Returns False when there is no such class."""
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.moe_offload.runtime import get_moe_offload_runtime

    cls = getattr(_comm, "MoECommMethod", None)
    if cls is None:
        return False
    if _is_tagged(getattr(cls, "fused_experts", None), PATCH_TAG) and _is_tagged(
            getattr(cls, "_maybe_apply_moe_offload_plan", None), PATCH_TAG):
        return True
    contracts = (
        _contract(_comm, "MoEFusedExpertsInput", fused_moe.MoEFusedExpertsInput),
        _contract(_comm, "MoEWeights", fused_moe.MoEWeights),
        _contract(_comm, "MoERoutingParams", fused_moe.MoERoutingParams),
        _contract(_comm, "MoEOffloadParams", fused_moe.MoEOffloadParams),
    )
    result_cls = getattr(_comm, "FusedExpertsResult", None) or fused_moe.FusedExpertsResult
    if not hasattr(cls, "_latchmoe_original_fused_experts"):
        cls._latchmoe_original_fused_experts = getattr(cls, "fused_experts", None)
        cls._latchmoe_original_maybe_apply = getattr(cls, "_maybe_apply_moe_offload_plan", None)
    original_fused = cls._latchmoe_original_fused_experts
    original_maybe_apply = cls._latchmoe_original_maybe_apply

    def _with_prepared_slot_weights(self, fused_experts_input, prepared_weights, *, offload_enabled=None,
                                    use_log2phy=True):
        self._latchmoe_slot_compute_handle = get_moe_offload_runtime().begin_slot_compute(prepared_weights)
        return fused_moe.with_slot_weights(fused_experts_input, prepared_weights, offload_enabled=offload_enabled,
                                           use_log2phy=use_log2phy, contracts=contracts)

    def _maybe_apply_moe_offload_plan(self, fused_experts_input):
        off = getattr(fused_experts_input, "offload", None)
        if off is None or not getattr(off, "enabled", False):
            return fused_experts_input
        runtime = get_moe_offload_runtime()
        prepared = _graph_capture_slot_weights(runtime, layer_id=int(off.layer_id))
        if prepared is not None:
            prepared.validate_backend_ready(expected_device_type=getattr(off, "expected_device_type", "cuda"))
            return self._with_prepared_slot_weights(fused_experts_input, prepared)
        if original_maybe_apply is not None:
            return original_maybe_apply(self, fused_experts_input)
        return fused_experts_input

    def fused_experts(self, fused_experts_input):
        off = getattr(fused_experts_input, "offload", None)
        if off is None or not getattr(off, "enabled", False):
            if original_fused is None:
                return fused_moe.run_fused_experts_contract(fused_experts_input, result_cls=result_cls)
            return original_fused(self, fused_experts_input)
        runtime = get_moe_offload_runtime()
        layer_id = int(off.layer_id)
        if runtime.consume_device_waves(layer_id=layer_id, topk_ids=fused_experts_input.topk_ids):
            # the seam left this overflow to the device planner: no host step
            fused_moe.check_supported_input(fused_experts_input)
            w = fused_experts_input.topk_weights
            out = fused_moe.run_overflow_prefill(
                runtime, layer_id=layer_id, hidden=fused_experts_input.hidden_states,
                topk_weights=w if w.dtype == torch.bfloat16 else w.to(torch.bfloat16),
                topk_ids=fused_experts_input.topk_ids.to(torch.int32).contiguous(),
                num_logical_experts=int(off.num_logical_experts), device_planned=True,
                add=getattr(fused_experts_input, "shared_output", None),
            )
            return result_cls(routed_out=out, before_dispatch_evt=None, before_gmm2_evt=None,
                              before_combine_evt=None, group_list_type=1, expert_tokens=None,
                              swiglu_limit=getattr(fused_experts_input, "swiglu_limit", None))
        stats = runtime.consume_prefill_route_stats_record(layer_id=layer_id, topk_ids=fused_experts_input.topk_ids)
        if stats is not None:
            # the stage op deferred an overflow: capacity waves, one combine
            fused_moe.check_supported_input(fused_experts_input)
            out = fused_moe.run_overflow_prefill(
                runtime, layer_id=layer_id, hidden=fused_experts_input.hidden_states,
                topk_weights=fused_experts_input.topk_weights, topk_ids=fused_experts_input.topk_ids,
                num_logical_experts=int(off.num_logical_experts), device_planned=False,
                add=getattr(fused_experts_input, "shared_output", None),
                token_counts_by_expert=dict(stats.token_counts_by_expert),
            )
            return result_cls(routed_out=out, before_dispatch_evt=None, before_gmm2_evt=None,
                              before_combine_evt=None, group_list_type=1, expert_tokens=None,
                              swiglu_limit=getattr(fused_experts_input, "swiglu_limit", None))
        overflow = runtime.decode_overflow_slot_weights(layer_id=layer_id,
                                                        n_pairs=int(fused_experts_input.topk_ids.numel()))
        prepared_input = self._maybe_apply_moe_offload_plan(fused_experts_input)
        try:
            return fused_moe.run_fused_experts_contract(prepared_input, result_cls=result_cls, record_events=True,
                                                        overflow=overflow)
        finally:
            handle = getattr(self, "_latchmoe_slot_compute_handle", None)
            self._latchmoe_slot_compute_handle = None
            runtime.end_slot_compute(handle)
            if overflow is not None:
                runtime.end_overflow_compute(layer_id)

    cls._with_prepared_slot_weights = _with_prepared_slot_weights
    cls._maybe_apply_moe_offload_plan = _tagged(_maybe_apply_moe_offload_plan, PATCH_TAG)
    cls.fused_experts = _tagged(fused_experts, PATCH_TAG)
    return True


@contextmanager
def moe_layer_context(layer):
    """The layer whose select_experts call is running (set by apply())."""
    prev = getattr(_layer_ctx, "layer", None)
    _layer_ctx.layer = layer
    try:
        yield
    finally:
        _layer_ctx.layer = prev


def _layer_id(layer) -> int | None:
    lid = getattr(layer, "layer_id", None)
    return None if lid is None or int(lid) < 0 else int(lid)


def _patch_select_experts(owner, name: str = "select_experts") -> bool:
    """Wrap owner.<name> (a module function or a static/class method) so that
    an injected top-k is returned for the current layer, and the ids of an
    offloaded layer go through the stage op."""
    from vllm_moe_offload_amd.ops.fused_moe import moe_seam_inject

    current = getattr(owner, name, None)
    if current is None:
        return False
    if _is_tagged(current, SELECT_TAG):
        return True
    original = current

    def select_experts(*args, **kwargs):
        layer = getattr(_layer_ctx, "layer", None)
        lid = _layer_id(layer) if layer is not None else None
        if lid is not None:
            injected = moe_seam_inject.peek_injected_topk(lid)
            if injected is not None:
                return injected
        weights, ids = original(*args, **kwargs)
        if lid is not None:
            from vllm_moe_offload_amd.moe_offload.runtime import get_moe_offload_runtime

            runtime = get_moe_offload_runtime()
            n_logical = int(kwargs.get("num_experts", getattr(layer, "num_logical_experts", -1)) or -1)
            if runtime.config.offload_stage_seam and runtime.should_use_fixed_slot_plan_for_layer(lid) and n_logical > 0:
                import torch

                from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_UNKNOWN

                torch.ops.vllm.moe_offload_stage(ids, lid, n_logical, PHASE_UNKNOWN)
        return weights, ids

    if isinstance(owner, type) and isinstance(owner.__dict__.get(name), staticmethod):
        setattr(owner, name, staticmethod(_tagged(select_experts, SELECT_TAG)))
    else:
        setattr(owner, name, _tagged(select_experts, SELECT_TAG))
    return True


def _patch_quant_method_apply(cls) -> bool:
    """Publish the layer to select_experts while cls.apply(self, layer, ...)
    runs."""
    current = getattr(cls, "apply", None)
    if current is None:
        return False
    if _is_tagged(current, SELECT_TAG):
        return True
    original = current

    def apply(self, layer, *args, **kwargs):
        with moe_layer_context(layer):
            return original(self, layer, *args, **kwargs)

    cls.apply = _tagged(apply, SELECT_TAG)
    return True


def _patch_quant_method_weights(cls) -> bool:
    """CPU-first create_weights and the registration after loading:
    create_weights makes host expert parameters for offloaded layers, and
    process_weights_after_loading registers every offloaded layer's host
    store and slot bank (then releases the originals when configured).
    Reference: patches/patch_fused_moe.py:4537-4576 and :4748-4790."""
    create = getattr(cls, "create_weights", None)
    process = getattr(cls, "process_weights_after_loading", None)
    if create is None or process is None:
        return False
    if _is_tagged(create, WEIGHTS_TAG) and _is_tagged(process, WEIGHTS_TAG):
        return True
    from vllm_moe_offload_amd.moe_offload.runtime import get_moe_offload_runtime
    from vllm_moe_offload_amd.moe_offload.cpu_first_loader import (
        ensure_moe_layer_id,
        maybe_create_unquantized_cpu_first_weights,
        maybe_process_unquantized_cpu_first_weights,
        maybe_register_unquantized_fixed_slot_weights,
    )

    original_create, original_process = create, process

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        ensure_moe_layer_id(layer)
        if maybe_create_unquantized_cpu_first_weights(
            self, layer, runtime=get_moe_offload_runtime(), num_experts=num_experts,
            hidden_size=hidden_size, intermediate_size_per_partition=intermediate_size_per_partition,
            params_dtype=params_dtype, extra_weight_attrs=extra_weight_attrs,
        ):
            return None
        return original_create(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                               params_dtype, **extra_weight_attrs)

    def process_weights_after_loading(self, layer):
        ensure_moe_layer_id(layer)
        rt = get_moe_offload_runtime()
        if maybe_process_unquantized_cpu_first_weights(self, layer, runtime=rt):
            return None
        result = original_process(self, layer)
        maybe_register_unquantized_fixed_slot_weights(layer, runtime=rt)
        return result

    if not _is_tagged(create, WEIGHTS_TAG):
        cls.create_weights = _tagged(create_weights, WEIGHTS_TAG)
    if not _is_tagged(process, WEIGHTS_TAG):
        cls.process_weights_after_loading = _tagged(process_weights_after_loading, WEIGHTS_TAG)
    return True


def _patch_engine_args_autoconfig(arg_utils=None) -> bool:
    """Wrap EngineArgs.create_engine_config so the final config keeps the stage
    op as a PIECEWISE splitting op (fail closed on FULL graph modes)."""
    from vllm_moe_offload_amd.plugin import ensure_moe_offload_splitting_op

    if arg_utils is None:
        try:
            arg_utils = importlib.import_module("vllm.engine.arg_utils")
        except Exception:
            return False
    engine_args = getattr(arg_utils, "EngineArgs", None)
    current = getattr(engine_args, "create_engine_config", None) if engine_args is not None else None
    if current is None:
        return False
    if _is_tagged(current, ENGINE_TAG):
        return True
    original = current

    def create_engine_config(self, *args, **kwargs):
        vllm_config = original(self, *args, **kwargs)
        comp = getattr(vllm_config, "compilation_config", None)
        if comp is not None and _stage_seam_enabled():
            ensure_moe_offload_splitting_op(comp)
            if os.environ.get("LATCHMOE_VERBOSE"):
                print("LATCHMOE_GRAPH_CONFIG cudagraph_mode=PIECEWISE splitting_op=vllm::moe_offload_stage", flush=True)
        return vllm_config

    engine_args.create_engine_config = _tagged(create_engine_config, ENGINE_TAG)
    return True


def _patch_graph_replay_profile(graph_mod=None, context_mod=None) -> bool:
    """Sample the host-side issue time of hipGraph replays (the first replay,
    then every N-th, N = VLLM_ASCEND_MOE_GRAPH_REPLAY_PROFILE_SAMPLE_RATE,
    default 1024) as graph_replay_issue events; nothing synchronizes the
    device.  Only replays count: capture and eager calls pass through.
    Reference: patches/patch_fused_moe.py:1603-1667."""
    try:
        graph_mod = graph_mod or importlib.import_module("vllm.compilation.cuda_graph")
        context_mod = context_mod or importlib.import_module("vllm.forward_context")
    except Exception:
        return False
    wrapper = getattr(graph_mod, "CUDAGraphWrapper", None)
    current = getattr(wrapper, "__call__", None) if wrapper is not None else None
    get_context = getattr(context_mod, "get_forward_context", None)
    if current is None or get_context is None:
        return False
    if _is_tagged(current, REPLAY_TAG):
        return True
    original = current

    def __call__(self, *args, **kwargs):
        ctx = get_context()
        mode = getattr(ctx, "cudagraph_runtime_mode", None)
        entry = (getattr(self, "concrete_cudagraph_entries", None) or {}).get(getattr(ctx, "batch_descriptor", None))
        if mode is None or mode != getattr(self, "runtime_mode", None) or getattr(entry, "cudagraph", None) is None:
            return original(self, *args, **kwargs)
        count = int(getattr(self, "_latchmoe_replay_calls", 0)) + 1
        self._latchmoe_replay_calls = count
        try:
            rate = max(1, int(os.environ.get("VLLM_ASCEND_MOE_GRAPH_REPLAY_PROFILE_SAMPLE_RATE", "1024")))
        except ValueError:
            rate = 1024
        if not (count == 1 or count % rate == 0):
            return original(self, *args, **kwargs)
        from time import perf_counter

        from vllm_moe_offload_amd.moe_offload.runtime import get_moe_offload_runtime

        start = perf_counter()
        out = original(self, *args, **kwargs)
        get_moe_offload_runtime()._record_profile_event(
            "graph_replay_issue", layer_id=None, start=start,
            payload={"profile_sample_rate": 1 if count == 1 else rate, "replay_call_index": count,
                     "runtime_mode": str(mode), "synchronizes_npu": False, "synchronizes_device": False},
        )
        return out

    wrapper.__call__ = _tagged(__call__, REPLAY_TAG)
    return True


def _stage_seam_enabled() -> bool:
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig

    cfg = MoeOffloadConfig.from_env()
    return bool(cfg.enabled and cfg.offload_stage_seam)


def apply_patches() -> dict[str, bool]:
    """Install every hook whose target the installed vLLM provides."""
    done = {"comm_method": False, "select_experts": False, "quant_apply": False, "quant_weights": False,
            "engine_args": False, "graph_replay_profile": False}
    for mod in ("vllm.model_executor.layers.fused_moe.moe_comm_method",
                "vllm_ascend.ops.fused_moe.moe_comm_method"):
        try:
            target = importlib.import_module(mod)
        except Exception:  # absent, or a vLLM build whose import fails
            continue
        done["comm_method"] |= _patch_moe_comm_method_runtime_hooks(target)
    try:
        layer_mod = importlib.import_module("vllm.model_executor.layers.fused_moe.layer")
    except Exception:
        layer_mod = None
    if layer_mod is not None:
        fused = getattr(layer_mod, "FusedMoE", None)
        if fused is not None:
            done["select_experts"] = _patch_select_experts(fused)
        method = getattr(layer_mod, "UnquantizedFusedMoEMethod", None)
        if method is not None:
            done["quant_apply"] = _patch_quant_method_apply(method)
            done["quant_weights"] = _patch_quant_method_weights(method)
    done["engine_args"] = _patch_engine_args_autoconfig()
    done["graph_replay_profile"] = _patch_graph_replay_profile()
    return done
