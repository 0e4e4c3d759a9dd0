"""The reference's ``CpuKVRunGather`` (cpu_kv_run_gather.py:8-17): the same
call as ``CpuKVGather`` with runs of consecutive source rows copied as one
block.  The reference keeps two natives that differ in a run threshold of 16
rows; ``tw_host_gather_kv`` coalesces every run, so both classes bind it, and
the outputs are the same bytes either way."""

from __future__ import annotations

from .cpu_kv_gather import CpuKVGather

__all__ = ["CpuKVRunGather"]


class CpuKVRunGather(CpuKVGather):
    """Hybrid run/row copy (bit-exact ``index_select`` of K and V)."""
