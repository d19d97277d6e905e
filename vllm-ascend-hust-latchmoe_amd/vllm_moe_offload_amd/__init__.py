"""vllm_moe_offload_amd: LatchMoE's slot-indexed fused-MoE hot path on MI355X.

Drop-in for the reference plugin's hot path (vllm_moe_offload_ascend): the
same vLLM general-plugin entry point, slot-bank / host-store / staging objects
and placement-plan adapter, with the router, permutation, grouped GEMM,
combine and staging executed by hand-written gfx950 HIP kernels
(liblatchmoe_hip.so, see native.py).

Reference: vllm_moe_offload_ascend/__init__.py:38-58 (register()).
"""

__all__ = ["register"]


def register() -> None:
    """Entry point called by vLLM's general-plugin loader in every process.

    Mirrors vllm_moe_offload_ascend.register (__init__.py:38-58): register the
    custom ops of the seam (router / stage / MLP) and install the fused-MoE
    hooks when vLLM is importable.  Idempotent.
    """
    from vllm_moe_offload_amd.plugin import register as _register

    _register()
