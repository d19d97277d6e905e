"""Slot-bank offload runtime: slot bank, host store, staging controller,
wave planner and placement-plan adapter (host side of the hot path)."""
