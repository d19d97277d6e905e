"""Installers of the slot-bank MoE seam into vLLM (best effort, idempotent)."""
