"""CPU oracle of the slot-indexed fused-MoE hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and plain Python for the small host-side
planners), the algorithm of the LatchMoE hot path so that the HIP kernels of
`vllm_moe_offload_amd` can be checked against it.  It is imported only by
`tests/`, by `__graft_entry__.smoke()` and by the `cpu_baseline` leg of
`bench.py`, and only as the checker or as the reported CPU baseline.  Product
code never imports it: the product path fails loudly when the HIP library is
missing.

Modules and the reference code each restates (paths relative to the LatchMoE
repository):
  bf16     bf16 round-to-nearest-even packing used by every module
  router   select_experts softmax / grouped-sigmoid top-k with renorm
           (ops/fused_moe/moe_router_op.py:72-125, patches/patch_fused_moe.py:597-632)
  permute  log2phy remap + npu_moe_init_routing_v2 stable sort and histogram
           (moe_offload/slot_mapping.py:116-140, patch_fused_moe.py:668-701)
  mlp      grouped SwiGLU MLP with f32 accumulation and the weighted combine
           (patch_fused_moe.py:3772-3774, 3342-3379; phase_split.py:1649-1656)
  slots    LRU fixed-slot staging with persistent log2phy
           (moe_offload/slot_bank.py:211-328, runtime.py:1636-1936)
  waves    canonical capacity-bounded wave planner, device pair planner,
           prefill async schedule (moe_offload/phase_split.py:479-766, 1224-1384)

Pinning (what checks each function against something other than itself) is
listed in each module's docstring; every function is pinned.
"""
