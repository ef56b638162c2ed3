"""Compile-time runtime support: the liveness memory planner and arena layout."""

from mdlc_amd.runtime.memory_planner import Buffer, MemoryPlan, plan_memory

__all__ = ["Buffer", "MemoryPlan", "plan_memory"]
