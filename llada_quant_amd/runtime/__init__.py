"""Execution of the packed expert path: the HIP library binding, residency, routing, fused_moe."""
