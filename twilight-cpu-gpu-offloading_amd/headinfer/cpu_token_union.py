"""Sorted CPU token union over a bounded membership array: the reference's
``CpuTokenUnion`` (cpu_token_union.py:6-23), backed by
``tw_host_token_union`` in ``libtwilight_host.so``.

``CpuTokenUnion(capacity)(positions, length)`` returns the ascending int64
union of the position lists, all of which must lie in ``[0, length)``;
``length`` must lie in ``[0, capacity]``.  Errors are the reference's
``ValueError``s.  The result owns its memory, so reusing the object cannot
change an earlier result."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _native

__all__ = ["CpuTokenUnion"]


class CpuTokenUnion:
    def __init__(self, capacity: int) -> None:
        self.members = np.zeros(int(capacity), dtype=np.uint8)
        self._fn = _native.host().tw_host_token_union

    def __call__(self, positions: list[torch.Tensor], length: int) -> torch.Tensor:
        if not 0 <= length <= self.members.size:
            raise ValueError("invalid union length")
        # one list at a time, dtype then range, as the reference checks them
        # (cpu_token_union.py:15-20): the first bad list decides the error
        lists = []
        for selected in positions:
            if selected.device.type != "cpu" or selected.dtype != torch.int64:
                raise ValueError("union expects CPU int64 indices")
            flat = selected.contiguous().reshape(-1)
            if flat.numel() and (int(flat.min()) < 0 or int(flat.max()) >= length):
                raise ValueError("selected position outside history")
            lists.append(flat)
        out = torch.empty(length, dtype=torch.int64)
        if length == 0:
            return out
        n = len(lists)
        ptrs = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in lists])
        sizes = np.array([t.numel() for t in lists] or [0], dtype=np.int64)
        count = self._fn(ptrs, sizes.ctypes.data, n, length, self.members.ctypes.data, out.data_ptr())
        if count == -2:
            raise ValueError("selected position outside history")
        if count < 0:
            raise ValueError("invalid union arguments")
        return out[:count].clone()
