"""vLLM general-plugin wiring: custom ops of the seam, the hooks and the
splitting-op contract.

register() is idempotent and safe to call in every vLLM process (API,
EngineCore, Worker).  It registers the custom ops, then installs the
fused-experts, router and EngineArgs hooks of patches/patch_fused_moe.py
where the installed vLLM provides their targets; the EngineArgs hook checks
the compilation config contract: the seam needs PIECEWISE graph mode with
vllm::moe_offload_stage among the splitting ops, and fails closed otherwise.

Reference: vllm_moe_offload_ascend/__init__.py:38-58 (register),
patches/patch_fused_moe.py:64-77 (_register_plugin_ops), :781-827
(apply_patches), :5339-5406 (_ensure_moe_offload_splitting_op).
"""

from __future__ import annotations

import os

_REGISTERED = False
STAGE_SPLITTING_OP = "vllm::moe_offload_stage"
PLUGIN_ENTRY_POINT = ("vllm.general_plugins", "moe_offload_ascend", "vllm_moe_offload_amd:register")


def register_plugin_ops() -> None:
    from vllm_moe_offload_amd.ops.fused_moe import moe_mlp_op, moe_offload_stage_op, moe_router_op

    moe_router_op.register()
    moe_offload_stage_op.register()
    moe_mlp_op.register()


INSTALLED_HOOKS: dict[str, bool] = {}


def register() -> None:
    global _REGISTERED
    if _REGISTERED:
        return
    register_plugin_ops()
    # the fused-experts, router and engine-config hooks, where the installed
    # vLLM provides their targets (nothing is patched without vLLM)
    from vllm_moe_offload_amd.patches.patch_fused_moe import apply_patches

    INSTALLED_HOOKS.update(apply_patches())
    _REGISTERED = True
    if os.environ.get("LATCHMOE_VERBOSE"):
        print("LATCHMOE_PLUGIN registered ops=moe_router,moe_router_indirect,moe_offload_stage,moe_mlp,moe_mlp_shared",
              flush=True)


def ensure_moe_offload_splitting_op(compilation_config) -> None:
    """Fail closed unless the graph mode is PIECEWISE and the stage op splits
    the graph (so staging runs eager between the two captured pieces)."""
    mode = getattr(compilation_config, "cudagraph_mode", None)
    mode_name = str(getattr(mode, "name", mode) or "").upper()
    if mode_name and "FULL" in mode_name and "PIECEWISE" not in mode_name:
        raise RuntimeError(
            f"slot-bank MoE offload requires PIECEWISE graph capture, got cudagraph_mode={mode_name}"
        )
    ops = getattr(compilation_config, "splitting_ops", None)
    if ops is None:
        compilation_config.splitting_ops = [STAGE_SPLITTING_OP]
        return
    if STAGE_SPLITTING_OP not in list(ops):
        ops = list(ops) + [STAGE_SPLITTING_OP]
        compilation_config.splitting_ops = ops
