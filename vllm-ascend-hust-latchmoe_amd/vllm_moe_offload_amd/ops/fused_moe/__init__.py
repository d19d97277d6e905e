"""vllm::moe_router, vllm::moe_offload_stage and vllm::moe_mlp on gfx950."""
