"""Bit-exact CPU K/V row copy into (pinned) staging: the reference's
``CpuKVGather`` (cpu_kv_gather.py:9-36), the host half of the gather + DMA
variant of the host path.

The reference compiles its ``.cpp`` with g++ into a temporary directory when
the object is built; here the native is part of ``libtwilight_host.so``,
built in-tree ahead of time, and a missing library raises instead of
compiling.  Arguments, validation order and error types are the reference's:
``gather(key, value, rows, out_key, out_value)`` with 2-D contiguous CPU
tensors and int64 rows, ``ValueError`` for a bad layout or an out-of-range
row, nothing to do for an empty row list.  The copy runs on
``torch.get_num_threads()`` OpenMP workers (the reference passes the same
count) and coalesces runs of consecutive rows into one ``memcpy``.
"""

from __future__ import annotations

import torch

from . import _native

__all__ = ["CpuKVGather"]


class CpuKVGather:
    """``out_key[i] = key[rows[i]]``, ``out_value[i] = value[rows[i]]``."""

    def __init__(self) -> None:
        self.library = _native.host()
        self.fn = self.library.tw_host_gather_kv

    def __call__(self, key: torch.Tensor, value: torch.Tensor, rows: torch.Tensor, out_key: torch.Tensor,
                 out_value: torch.Tensor) -> None:
        tensors = (key, value, rows, out_key, out_value)
        if any(t.device.type != "cpu" or not t.is_contiguous() for t in tensors):
            raise ValueError("CPU contiguous tensors required")
        if key.ndim != 2 or key.shape != value.shape or key.dtype != value.dtype:
            raise ValueError("invalid source layout")
        if rows.ndim != 1 or rows.dtype != torch.int64:
            raise ValueError("int64 row indices required")
        if out_key.shape != (rows.numel(), key.shape[1]) or out_key.shape != out_value.shape:
            raise ValueError("invalid output layout")
        if out_key.dtype != key.dtype or out_value.dtype != key.dtype:
            raise ValueError("dtype mismatch")
        if rows.numel() == 0:
            return
        rc = self.fn(key.data_ptr(), value.data_ptr(), out_key.data_ptr(), out_value.data_ptr(), rows.data_ptr(),
                     rows.numel(), key.shape[0], key.shape[1] * key.element_size(), torch.get_num_threads())
        if rc:
            raise ValueError("row index out of bounds")
